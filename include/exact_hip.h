/* exact_hip.h - C ABI of the MI355X (gfx950) exact integer forward path.
 *
 * Plain C: device pointers, sizes and a hipStream_t (passed as void*), no torch types.
 * Every entry point validates shapes on the host, launches on the given stream, never
 * allocates device memory and never synchronises, so a caller may capture it in a HIP graph.
 * Return value: EXACT_OK (0) or one of the EXACT_E_* codes below (nothing was launched unless
 * the code is EXACT_E_LAUNCH).
 *
 * Data formats
 *   activations  int64 Q16, row-major (R, D)
 *   xq           quantised rows from qrow: int16 (bits 8..15) or int8 (bits <= 7), shifts s int32 (R)
 *   packed linear (N outputs, K inputs, K % 128 == 0, nbs = ceil(N / 64), G = K / 128), tiles in
 *   group-major order T = g * nbs + nb:
 *       wp int8  [G][nbs][8][64][16]  wp[(T*8 + j)*1024 + l*16 + b] = W[n = nb*64+l][k = g*128+j*16+b]
 *       mp int16 [G][nbs][64]         mp[T*64 + l] = M[g][n]   (positive group-128 scales)
 *     One 8 KiB tile holds 64 output rows x one 128-wide group; rows n >= N are zero. A buffer of Ntot
 *     rows may stack several linears of the same K (fused q|k|v, gate|up), each at a row offset n_off
 *     that is a multiple of 64.
 *   t            int64 (R, N): t = sum_g acc_g * M_g, acc_g = sum_{k in g} xq[k] * W[n][k] (exact)
 *   tables       EXP_T (10242 x Q24) and SILU_T / SIG_T (8194 x Q16) as int32 device arrays
 */
#ifndef EXACT_HIP_H
#define EXACT_HIP_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define EXACT_OK 0
#define EXACT_E_ARG 1        /* null pointer, bad size or shape */
#define EXACT_E_UNSUPPORTED 2 /* size outside what the kernels handle (e.g. K % 128, R too large) */
#define EXACT_E_LAUNCH 3     /* the HIP launch reported an error */

/* Library version (major*10000 + minor*100 + patch). */
int exact_version(void);

/* Last HIP error string seen by the library (for diagnostics; not thread-safe). */
const char* exact_last_error(void);

/* ---- weights ------------------------------------------------------------------------------------
 * Seeded synthetic linear written straight into the packed layout. W[n][k] for logical index
 * i = n*K + k is -127 + #{j : thr[j] <= (splitmix64(key_w, i) >> 32)} with the 254 thresholds of a
 * rounded, clipped N(0, 40^2); M[g][n] = m_lo + (((splitmix64(key_m, n*G + g) >> 32) * (m_hi - m_lo)) >> 32).
 * No counterpart in the reference (it quantises downloaded float checkpoints, exact_llm.py:82-88);
 * this is the seeded integer artifact of SPEC.md:7-12 generated on the device. */
int exact_synth_linear(uint64_t key_w, uint64_t key_m, int32_t m_lo, int32_t m_hi, const uint32_t* thr,
                       int8_t* wp, int16_t* mp, int32_t N, int32_t K, int32_t n_off, int32_t Ntot, void* stream);

/* out[i] = lo + (((splitmix64(key, i) >> 32) * (hi - lo)) >> 32), i < n (gains, biases). */
int exact_synth_vector(uint64_t key, int64_t lo, int64_t hi, int64_t* out, int64_t n, void* stream);

/* Repack a (K, N) row-major int8 weight (QLin.w layout, exact_llm.py:85) and (G, N) int16 scales
 * (GQLin.M, speed_fair_kaggle.py:717) into the packed layout. Replaces TLinG's wT = w.T.contiguous()
 * and Mg = M.T (speed_fair_kaggle.py:730-731). */
int exact_pack_linear(const int8_t* w_kn, const int16_t* m_gn, int8_t* wp, int16_t* mp,
                      int32_t N, int32_t K, int32_t n_off, int32_t Ntot, void* stream);

/* Repack (G, N) int16 values into the scale layout of exact_pack_linear alone: the high plane mh of wide
 * scales (below). */
int exact_pack_scales(const int16_t* m_gn, int16_t* mp, int32_t N, int32_t K, int32_t n_off, int32_t Ntot,
                      void* stream);

/* ---- linears ------------------------------------------------------------------------------------
 * Group scales: mh == NULL: M = mp, int16 in [0, 2^15). Wide scales (M < 2^30; quantised checkpoints give
 * up to about 2^21, the reference asserts M < 2^27, group128_quality_kaggle.py:419): M = mh * 2^15 + mp
 * with the low plane mp in [0, 2^15) and the high plane mh packed by exact_pack_scales.
 *
 * Exact group-128 GEMV for decode, R <= 15 (int16 x) or 16 (int8 x) rows: t[r][n] = sum_g acc_g * M[g][n].
 * abits = 15: x is int16 (xq from qrow(x, 15), the spec); abits = 7: x is int8 (exact_torch A8 mode).
 * Replaces the reference's exact::gemv op and its CUDA kernel gemv_g128_v2
 * (experiments/speed_fair_kaggle.py:656-702) and TLinG's R == 1 branch (:735-738), extended to R rows. */
int exact_gemv_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t,
                    int32_t R, int32_t N, int32_t K, void* stream);

/* Accumulating form: t[r][n] += sum_g acc_g * M[g][n]. No counterpart in the reference; used by fused
 * decode steps whose consumer kernels leave t zeroed after reading it, so no zero-fill launch is needed. */
int exact_gemv_g128_acc(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t,
                        int32_t R, int32_t N, int32_t K, void* stream);

/* The reference's exact::gemv on its own tensors, with no repacking: out[n] = sum_g (sum_{k in g} x[k] *
 * wT[n][k]) * Mg[n][g] for one int16 row x (K,), the row-major int8 weight wT (N, K) (TLinG.wT, each output's
 * K weights contiguous) and int64 group scales Mg (N, G), G = K / 128; int64 products and sums wrap like the
 * reference's. out (N,) int64 is written whole. K % 128 != 0 or x / wT not 16-byte aligned (Mg, out 8-byte)
 * return 2. Replaces the custom op exact::gemv and its kernel gemv_g128_v2
 * (experiments/speed_fair_kaggle.py:656-702), called by TLinG for one row (:738). */
int exact_gemv(const int16_t* x, const int8_t* wT, const int64_t* Mg, int64_t* out, int32_t N, int32_t K, void* stream);

/* Residual + RMSNorm + qrow fused into the int16 GEMV that consumes them (decode rows, R <= 2, K <= 6144):
 * t[r] += qrow(irms(x, g), 15) . W with x = x_in + round_shift(res_t, 28 - res_s[r]) (res_t may be NULL). Every
 * block normalises the rows itself (exact_llm.py:41-46, 100-106) while its first weight tiles load; block 0 writes
 * x to x_out (NULL: not written; must not alias x_in or res_t, which the other blocks still read), the row shifts
 * s_out[r] and, when xq_out is given, the quantised int16 rows. Replaces exact_rmsnorm_qrow + exact_gemv_g128_acc
 * (IntModel.__call__'s residual add, irms and linear, exact_llm.py:166-169, 177-179; TLinG, speed_fair_kaggle.py:735-738)
 * with one launch. */
int exact_gemv_g128_norm_acc(const int64_t* x_in, int64_t* x_out, const int64_t* res_t, const int32_t* res_s,
                             const int64_t* g, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t,
                             int32_t* s_out, int16_t* xq_out, int32_t R, int32_t N, int32_t K, void* stream);

/* Waves per block that exact_gemv_g128_norm_acc launches for R rows of an N x K linear on cus compute units (cus <= 0:
 * the current device's): 8 when the rows are wider than 1024 and the group-split tasks fit one round of 8-wave blocks,
 * or do with the split capped at no fewer than 8 parts (each CU then normalises the rows once), else 4; 0 for sizes the launch refuses. A host-side query (no launch), so
 * a caller choosing between the fused norm and a separate norm launch reads the kernel's own split. No counterpart in
 * the reference. */
int exact_gemv_g128_norm_acc_blockwaves(int32_t R, int32_t N, int32_t K, int32_t cus);

/* Exact group-128 GEMM for prefill (any R): same output as exact_gemv_g128. Up to 15 rows (A16) or 16 rows (A8)
 * run on the GEMV kernel, more rows on the MFMA GEMM kernels. Wide scales (mh != NULL): int8 rows at any R; int16
 * rows run as GEMV row chunks of 15 up to 45 rows, and above that 2 is returned (exact_gemm_g128_a16 covers them).
 * Replaces TLinG's R > 1 fp64 bmm branch (speed_fair_kaggle.py:739-742) and TLin._acc's
 * torch._int_mm A16/A8 passes (exact_torch.py:94-119). */
int exact_gemm_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t,
                    int32_t R, int32_t N, int32_t K, void* stream);

/* exact_gemm_g128 for a t that holds zeros on entry (the model's consumer kernels leave their totals so): the
 * K-split and row-chunk paths add into t instead of launching a clear first. No counterpart in the reference,
 * whose torch GEMMs allocate their outputs. */
int exact_gemm_g128_zeroed(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                           int64_t* t, int32_t R, int32_t N, int32_t K, void* stream);

/* qrow fused into the GEMV that consumes it: t += qrow(xs, abits) . W (t holds zeros or a running total), where
 * row r of xs (int64, ldx apart) is quantised with s = max(max_i part[r * nparts + i] - abits, 0) and
 * part holds the producer's bit lengths of max |xs| over slices of the row (exact_attention's per-head
 * obits, exact_swiglu_qrow's slice bit lengths); s_out[r] = s. Replaces exact_quant_rows + exact_gemv_g128_acc
 * (qrow, exact_llm.py:41-46; TLinG, speed_fair_kaggle.py:735-738) with one launch. R <= 15 (abits 15) or
 * 16 (abits 7), nparts <= 1024; returns 2 when a wave's share of a row exceeds 512 columns (the GEMV's group
 * split leaves 4 groups or fewer per wave at the decode shapes) or the slices of a block 64 KiB of LDS.
 * zero (optional): zero_n int64 the launch also clears (a buffer whose readers have finished, e.g. the q|k|v
 * totals exact_attention_qkv leaves in place), so no separate clear is launched. */
int exact_gemv_g128_qrow_acc(const int64_t* xs, int64_t ldx, const int32_t* part, int32_t nparts, int32_t abits,
                             const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int32_t* s_out,
                             int32_t R, int32_t N, int32_t K, int64_t* zero, int64_t zero_n, void* stream);

/* The gate|up GEMV with the SwiGLU in its epilogue, for decode rows (R <= 4, int16 x): the packed linear (N = 2I)
 * holds the gate rows [0, I) and the up rows [I, 2I); with t = x . W (never stored unless t is given),
 * g = rs(t[r][n], 28 - s[r]), u = rs(t[r][I + n], 28 - s[r]) and h[r][n] = round_shift(isilu(g) * u, 16), as
 * exact_swiglu_qrow with xq NULL; part[r * (I / 32) + b] = bit length of max |h[r][32 b .. 32 b + 32)|, for
 * exact_gemv_g128_qrow_acc (nparts = I / 32) to quantise. t (optional, (R, 2I)): receives the gate|up totals
 * (overwritten, for a trace). I % 64 == 0, K % 128 == 0. Replaces exact_gemv_g128_acc + exact_swiglu_qrow
 * (exact_llm.py:179; TLinG, speed_fair_kaggle.py:735-738; isilu exact_llm.py:118-122) with one launch that adds no
 * atomics. */
int exact_gemv_g128_swiglu(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh, const int32_t* s,
                           const int32_t* silu, int64_t* h, int32_t* part, int64_t* t, int32_t R, int32_t I, int32_t K,
                           void* stream);

/* exact_gemv_g128_swiglu on rows the launch normalises itself, as exact_gemv_g128_norm_acc (decode rows, R <= 2,
 * K <= 8192; above 2048 I a multiple of 128 or I / 64 at most the CU count): every block computes x = x_in + round_shift(res_t, 28 - res_s[r]) (res_t may be NULL) and
 * xq, s = qrow(irms(x, g), 15) while its first weight tiles load, then the SwiGLU GEMV on xq with those row shifts.
 * Block 0 writes x to x_out (NULL: not written; must not alias x_in or res_t) and s to s_out. h, part and t as
 * exact_gemv_g128_swiglu. Replaces exact_rmsnorm_qrow + exact_gemv_g128_acc + exact_swiglu_qrow
 * (exact_llm.py:41-46, 100-106, 178-179; speed_fair_kaggle.py:735-738) with one launch. */
int exact_gemv_g128_norm_swiglu(const int64_t* x_in, int64_t* x_out, const int64_t* res_t, const int32_t* res_s,
                                const int64_t* g, const int8_t* wp, const int16_t* mp, const int16_t* mh, int32_t* s_out,
                                const int32_t* silu, int64_t* h, int32_t* part, int64_t* t, int32_t R, int32_t I,
                                int32_t K, void* stream);

/* MoE expert GEMM on the matrix cores, grouped over the chunks exact_moe_dispatch wrote with chunk_rows = 128
 * (int16 x) or 256 (int8 x): for every chunk c < nchunks[0], rows p = chunk_p0[c] .. + chunk_n[c] of the
 * dispatched pairs, t[p] = x[row_map[p]] . W_e with e = chunk_e[c] (row_map NULL: x row p), expert e's packed
 * linear at wp + e * w_stride, mp + e * m_stride. int16 x runs as interleaved digit rows (as
 * exact_gemm_g128_a16) and needs colterm (NE, N) = each expert's sum_g colsum_g M_g. x8: workspace of 2 P K
 * (int16) or P K (int8, with row_map) bytes. max_chunks: the length of the chunk arrays (launch size).
 * Replaces the per-expert loop of MoEInt.moe (moe_exact_kaggle.py:460-464) for prefill-sized pair counts. */
int exact_gemm_g128_experts(const void* x, int32_t abits, const int32_t* row_map, const int8_t* wp, const int16_t* mp,
                            int64_t w_stride, int64_t m_stride, const int64_t* colterm, int8_t* x8, const int32_t* chunk_e,
                            const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks,
                            int64_t* t, int32_t P, int32_t N, int32_t K, void* stream);

/* The int16 (A16) GEMM on the int8 matrix cores as interleaved digit rows: x is split into rows
 * x8[2r] = x[r] >> 8 and x8[2r + 1] = (x[r] & 255) - 128 (exact_torch.py:101-102), the A8 GEMM runs on the
 * 2R digit rows, and each output row combines its pair: t[r] = 256 T[2r] + T[2r + 1] + 128 colterm.
 * colterm[n] = sum_g (sum_{k in g} W[k][n]) * M[g][n]: exact_gemv_g128 of an all-ones int8 row (A8) gives it,
 * once per linear. x8: caller workspace of 2 R K bytes (16-byte aligned). Same output as exact_gemm_g128
 * with abits 15; 2 R K < 2^32. Up to 48 rows run as GEMV row chunks of 16 (colterm replaces the GEMV's
 * all-ones row; x8 is not used then). */
int exact_gemm_g128_a16(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh, const int64_t* colterm,
                        int8_t* x8, int64_t* t, int32_t R, int32_t N, int32_t K, void* stream);

/* exact_gemm_g128_a16 for a t that holds zeros on entry (as exact_gemm_g128_zeroed). */
int exact_gemm_g128_a16_zeroed(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                               const int64_t* colterm, int8_t* x8, int64_t* t, int32_t R, int32_t N, int32_t K,
                               void* stream);

/* The int16-row GEMM from digit rows a producer already wrote (exact_rmsnorm_qrow, exact_swiglu_qrow or
 * exact_quant_rows with x8): x8 holds 2R int8 rows (x8[2r] = x[r] >> 8, x8[2r + 1] = (x[r] & 255) - 128), so
 * no split launch runs. zeroed != 0: t holds zeros on entry (as exact_gemm_g128_zeroed). Results equal
 * exact_gemm_g128_a16's on the int16 rows (exact_torch.py:101-102). */
int exact_gemm_g128_digits(const int8_t* x8, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                           const int64_t* colterm, int64_t* t, int32_t R, int32_t N, int32_t K, int32_t zeroed,
                           void* stream);

/* Group epilogue y = round_shift(t, 28 - s[r]) + b[n] (b may be NULL)
 * (speed_fair_kaggle.py:725,743; SPEC.md:18). */
int exact_requant_group(const int64_t* t, const int32_t* s, const int64_t* b, int64_t* y,
                        int32_t R, int32_t N, void* stream);

/* Per-channel epilogue with the per-row overflow drop rule: y may alias acc
 * (exact_llm.py:93-96; speed_fair_kaggle.py:745-746; SPEC.md:28). */
int exact_requant_channel(const int64_t* acc, const int32_t* s, const int64_t* M, int32_t Mbits,
                          const int64_t* b, int64_t* y, int32_t R, int32_t N, void* stream);

/* ---- integer nonlinearities ---------------------------------------------------------------------- */
/* Per-row quantiser qrow(x, bits) (exact_llm.py:41-46): xq int16 for bits >= 8, int8 for bits <= 7. */
int exact_qrow(const int64_t* x, int32_t bits, void* xq, int32_t* s, int32_t R, int32_t K, void* stream);

/* Integer RMSNorm alone, y = irms(x, g) (exact_llm.py:100-106). */
int exact_irms(const int64_t* x, const int64_t* g, int64_t* y, int32_t R, int32_t D, void* stream);

/* Fused residual + irms + qrow: if res_t != NULL, x += round_shift(res_t, 28 - res_s[r]) (written back
 * to x); then xq, s = qrow(irms(x, g), bits). Covers exact_llm.py:177-178 (o-proj residual, post-norm),
 * :179-180/166 (down-proj residual, next input norm) and the final norm before the head.
 * clear_t != 0 leaves res_t zeroed after reading it (ready for the next accumulating GEMV).
 * x8 (optional, bits >= 8): also the interleaved int8 digit rows of xq (2R rows: x8[2r] = xq[r] >> 8,
 * x8[2r + 1] = (xq[r] & 255) - 128), which exact_gemm_g128_digits takes. */
int exact_rmsnorm_qrow(int64_t* x, int64_t* res_t, const int32_t* res_s, const int64_t* g,
                       int32_t bits, void* xq, int32_t* s, int32_t R, int32_t D, int32_t clear_t, int8_t* x8,
                       void* stream);

/* SwiGLU on a fused gate|up total: g = rs(t[r][n], 28 - s[r]), u = rs(t[r][I + n], 28 - s[r]),
 * h = round_shift(isilu(g) * u, 16); xq, sq = qrow(h, bits). h: optional int64 (R, I) scratch for the
 * SwiGLU values; when NULL they may be written over t's gate half. t is left zeroed when clear_t != 0,
 * and is left as it was when clear_t == 0 and h is given (the totals stay readable, e.g. for a trace).
 * part: int32 workspace of R * ceil(I / 1024) slice bit lengths. xq may be NULL when h is given: then only h and
 * part are produced (bit length of max |h| per 1024-column slice), for exact_gemv_g128_qrow_acc to quantise.
 * x8 (optional, with xq, bits >= 8): xq's digit rows too, as exact_rmsnorm_qrow.
 * (exact_llm.py:179; isilu exact_llm.py:118-122). */
int exact_swiglu_qrow(int64_t* t, const int32_t* s, const int32_t* silu_t, int32_t bits, void* xq,
                      int32_t* sq, int32_t* part, int32_t R, int32_t I, int32_t clear_t, int64_t* h, int8_t* x8,
                      void* stream);

/* qrow with the row maximum supplied in parts (a producer kernel wrote part[r * nparts + i] =
 * bitlen(max |src| over its slice i of row r)): s = max(max_i part - bits, 0), xq = clip(rs(src, s))
 * (exact_llm.py:41-46; bitlen of the row max = max of the slice bit lengths). src rows are ld apart;
 * clear != 0 leaves src zeroed. x8 (optional, bits >= 8): xq's digit rows too, as exact_rmsnorm_qrow.
 * zero (optional): zero_n int64 the launch also clears (a buffer whose readers have finished, e.g. the q|k|v
 * totals exact_attention_qkv leaves in place). */
int exact_quant_rows(int64_t* src, int64_t ld, const int32_t* part, int32_t nparts, int32_t bits, void* xq,
                     int32_t* s, int32_t R, int32_t K, int32_t clear, int8_t* x8, int64_t* zero, int64_t zero_n,
                     void* stream);

/* Elementwise LUT nonlinearities on int64 arrays (isilu exact_llm.py:118-122; isig moe_exact_kaggle.py:420-424). */
int exact_isilu(const int64_t* x, const int32_t* silu_t, int64_t* y, int64_t n, void* stream);
int exact_isig(const int64_t* x, const int32_t* sig_t, int64_t* y, int64_t n, void* stream);

/* Integer softmax rows over the first n_valid[r] entries (all if n_valid == NULL) -> Q20
 * (exact_llm.py:109-115). */
int exact_isoftmax(const int64_t* sc, const int32_t* n_valid, const int32_t* exp_t, int64_t* p,
                   int32_t R, int32_t N, void* stream);

/* ---- attention ------------------------------------------------------------------------------------
 * KV cache (per layer): kq int16 [B][KV][Smax][hd], sk int32 [B][KV][Smax], v int64 [B][KV][Smax][hd].
 * Row r of a call belongs to cache slot slot[r] at position pos[r].
 *
 * q/k/v epilogue: y = rs(t, 28 - s[r]) + b for the fused q|k|v total (N = (H + 2 KV) * hd); RoPE on q and
 * k with the Q16 tables at pos[r]; k rows quantised per head (qrow 15) into the cache, v stored as is;
 * q rows quantised per head into qq (R, H, hd) int16 and sq (R, H); clear_t != 0 leaves t zeroed.
 * (exact_torch.py:144-151; GraphDecoder._step speed_fair_kaggle.py:614-619). */
int exact_qkv_rope_cache(int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                         const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* qq,
                         int32_t* sq, int16_t* kq, int32_t* sk, int64_t* v, int32_t R, int32_t H,
                         int32_t KV, int32_t hd, int32_t Smax, int32_t clear_t, void* stream);

/* Integer attention of R query rows against the cache, keys 0..pos[r] of slot[r]:
 * sc = rs((qq . kq) * INV, 32 - sq - sk); p = isoftmax(sc) (Q20); out = rs(p . v, 20), out (R, H*hd) int64.
 * (exact_llm.py:170-176; exact_torch.py:162-166; speed_fair_kaggle.py:620-624). Used for decode and,
 * with pos[r] = p0 + r, for causal prefill. obits (optional, R * H): bit length of max |out| per head,
 * the parts that exact_quant_rows takes for the o-projection input. */
int exact_attention(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                    const int64_t* v, const int32_t* slot, const int32_t* pos, const int32_t* exp_t,
                    int64_t* out, int32_t* obits, int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t Smax,
                    int32_t INV, void* stream);

/* exact_qkv_rope_cache followed by exact_attention in one launch, for decode rows that each own their
 * (slot, position): one row, or rows of different sequences (rows of one sequence in one pass read each
 * other's new keys and take the two launches). Same results, cache contents and obits; the quantised
 * queries stay on chip (no qq / sq) and t is left unchanged. Replaces the per-layer q/k/v epilogue + RoPE +
 * cache write + attention of exact_llm.py:170-176 / speed_fair_kaggle.py:603-624 at decode. exp_t 16-byte
 * aligned (staged into LDS). */
int exact_attention_qkv(const int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                        const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq, int32_t* sk,
                        int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int32_t R, int32_t H,
                        int32_t KV, int32_t hd, int32_t Smax, int32_t INV, void* stream);

/* exact_attention_qkv with obn (1, 2 or 4) obits entries per head: obits[(r H + h) obn + i], whose max is the
 * head's bit length (exact_quant_rows / exact_gemv_g128_qrow_acc take them with nparts = H obn). With obn > 1
 * the launch may split each head's p.V over up to obn blocks that each write a slice of the head's dimensions
 * and the bit length of that slice (short caches, while the blocks fit one round). Results identical to
 * exact_attention_qkv; obn = 1 is that entry point. No counterpart in the reference, whose attention
 * (exact_llm.py:170-176) returns the whole output and leaves its row maximum to qrow (exact_llm.py:41-46). */
int exact_attention_qkv_split(const int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                              const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq, int32_t* sk,
                              int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int32_t obn, int32_t R,
                              int32_t H, int32_t KV, int32_t hd, int32_t Smax, int32_t INV, void* stream);

/* The same attention for the prefill of one sequence on the matrix cores: R query rows of cache slot `slot`
 * at increasing positions pos[r] (< nkeys), against keys 0..pos[r]; results identical to exact_attention
 * (exact_llm.py:170-176; exact_torch.py:162-166). q.k runs on int8 digit products of the int16 q and k
 * (exact in int32), p.v on balanced int8 digits of p (Q20) and v, summed per digit shift in int32 and
 * combined modulo 2^64 like the reference's int64 product. hd = 128 and nkeys <= 32768 (otherwise
 * EXACT_E_UNSUPPORTED). work: device memory of at least exact_attention_prefill_workspace(R, H, KV, hd, nkeys)
 * bytes, 256-byte aligned (digit copies of the slot's k and v, per-row softmax statistics); exp_t 16-byte
 * aligned. */
int64_t exact_attention_prefill_workspace(int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t nkeys);
int exact_attention_prefill(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                            const int64_t* v, int32_t slot, const int32_t* pos, const int32_t* exp_t, int64_t* out,
                            int32_t* obits, void* work, int64_t work_bytes, int32_t R, int32_t H, int32_t KV,
                            int32_t hd, int32_t Smax, int32_t nkeys, int32_t INV, void* stream);

/* ---- mixture of experts (MoEInt.moe, moe_exact_kaggle.py:454-467) ------------------------------------
 * Router: logits = rs(t[r][0..NE), 28 - s[r]) (t rows ld apart, from the router linear); p = isoftmax over all
 * NE experts (Q20); the k experts with the largest p, ties to the lower index (np.argsort(-p,
 * kind="stable")[:k], moe_exact_kaggle.py:457). Writes p_sel, e_sel (R, k) in rank order. With gate_col >= 0
 * the row also carries the shared expert's gate logit (router and gate linear fused in one GEMV):
 * gate[r] = isig(rs(t[r][gate_col], 28 - s[r])) (moe_exact_kaggle.py:465-467). clear_t != 0 leaves t zeroed. */
int exact_router_topk(int64_t* t, int32_t ld, const int32_t* s, const int32_t* exp_t, int64_t* p_sel, int32_t* e_sel,
                      int32_t gate_col, const int32_t* sig_t, int64_t* gate, int32_t R, int32_t NE, int32_t k,
                      int32_t clear_t, void* stream);

/* Dispatch: the P = R*k pairs q = r*k + j grouped by expert (row order inside an expert), replacing the
 * per-expert Python loop `rows = nonzero(sel == e)` (moe_exact_kaggle.py:459-463). Outputs: pidx[q] = position
 * of pair q; pair_row[p] = its token row; s_pair[p] = s[row]; chunks of <= chunk_rows pairs of one expert
 * (chunk_e, chunk_p0, chunk_n; count in nchunks[0]; at most min(P, ceil(P/chunk_rows) + NE) chunks). */
int exact_moe_dispatch(const int32_t* e_sel, const int32_t* s, int32_t* pidx, int32_t* pair_row, int32_t* s_pair,
                       int32_t* chunk_e, int32_t* chunk_p0, int32_t* chunk_n, int32_t* nchunks, int32_t R,
                       int32_t NE, int32_t k, int32_t chunk_rows, void* stream);

/* Decode rows: exact_router_topk followed by exact_moe_dispatch in one launch (one wave), with the same arguments and
 * outputs as the two. No counterpart in the reference (its router and its per-expert loop are separate steps,
 * moe_exact_kaggle.py:456-463); for routers of at most 64 experts and at most 64 (row, expert) pairs, otherwise
 * EXACT_E_UNSUPPORTED (call the two entry points). */
int exact_moe_route(int64_t* t, int32_t ld, const int32_t* s, const int32_t* exp_t, int64_t* p_sel, int32_t* e_sel,
                    int32_t gate_col, const int32_t* sig_t, int64_t* gate, int32_t R, int32_t NE, int32_t k, int32_t clear_t,
                    int32_t* pidx, int32_t* pair_row, int32_t* s_pair, int32_t* chunk_e, int32_t* chunk_p0, int32_t* chunk_n,
                    int32_t* nchunks, int32_t chunk_rows, void* stream);

/* Expert GEMV: for every chunk, t[p] += x[row_map ? row_map[p] : p] . W_e for its pairs p, with expert e's
 * packed linear at wp + e*w_stride, mp + e*m_stride (bytes / int16 elements). chunk_n <= 15 (abits 15) or
 * 16 (abits 7). The per-expert gate/up and down linears of MoEInt.moe (moe_exact_kaggle.py:461-462). */
int exact_gemv_g128_experts(const void* x, int32_t abits, const int32_t* row_map, const int8_t* wp,
                            const int16_t* mp, int64_t w_stride, int64_t m_stride, const int32_t* chunk_e,
                            const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks,
                            int32_t max_chunks, int64_t* t, int32_t N, int32_t K, void* stream);

/* Decode expert gate|up GEMV with the SwiGLU as its epilogue (int16 rows, chunks of at most 4 pairs, as
 * exact_moe_dispatch writes them with chunk_rows <= 4; chunk = that size, refused above 4): for every pair p of
 * every chunk, the expert's gate|up totals of x[row_map[p]] (the 2 I rows at wp + e*w_stride: gate rows [0, I),
 * up rows [I, 2 I)) and h[p][i] = rs(isilu(rs(g_i, 28 - s_pair[p])) * rs(u_i, 28 - s_pair[p]), 16), the bit length
 * of max |h| per 32 columns in part[p * (I / 32) + i / 32]. I % 64 == 0. Replaces exact_gemv_g128_experts +
 * exact_swiglu_qrow for the expert MLP's first half (moe_exact_kaggle.py:461-462; exact_llm.py:179). */
int exact_gemv_g128_experts_swiglu(const int16_t* x, const int32_t* row_map, const int8_t* wp, const int16_t* mp,
                                   int64_t w_stride, int64_t m_stride, const int32_t* chunk_e, const int32_t* chunk_p0,
                                   const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks, int32_t chunk,
                                   const int32_t* s_pair, const int32_t* silu, int64_t* h, int32_t* part, int32_t I,
                                   int32_t K, void* stream);

/* Decode expert down GEMV on the int64 SwiGLU values xs (row p at xs + p * ldx) quantised in the launch: each pair's
 * shift s_out[p] = max(max_i part[p * nparts + i] - 15, 0) (qrow, exact_llm.py:41-46) and t[p] += qrow(xs[p]) . W_e
 * for the dispatched chunks (chunk as exact_gemv_g128_experts_swiglu). Replaces exact_swiglu_qrow's quantisation +
 * exact_gemv_g128_experts for the expert MLP's second half (moe_exact_kaggle.py:461-462). */
int exact_gemv_g128_experts_qrow_acc(const int64_t* xs, int64_t ldx, const int32_t* part, int32_t nparts,
                                     const int8_t* wp, const int16_t* mp, int64_t w_stride, int64_t m_stride,
                                     const int32_t* chunk_e, const int32_t* chunk_p0, const int32_t* chunk_n,
                                     const int32_t* nchunks, int32_t max_chunks, int32_t chunk, int64_t* t,
                                     int32_t* s_out, int32_t N, int32_t K, void* stream);

/* MoE decode (R <= 2 rows): exact_gemv_g128_experts_swiglu (the routed experts, expert linears ewp/emp of I = EI) and
 * exact_gemv_g128_swiglu on the same rows x (the shared expert, swp/smp/smh of I = SI, row shifts s) in one launch:
 * eh/epart and sh/spart as those two entries write them; K is both linears' K. No counterpart in the reference, whose
 * MoE layer runs the experts and the shared expert one after the other (MoEInt.moe, moe_exact_kaggle.py:454-467). */
int exact_moe_swiglu_pair(const int16_t* x, const int32_t* row_map, const int8_t* ewp, const int16_t* emp,
                          int64_t w_stride, int64_t m_stride, const int32_t* chunk_e, const int32_t* chunk_p0,
                          const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks, int32_t chunk,
                          const int32_t* s_pair, const int32_t* silu, int64_t* eh, int32_t* epart, int32_t EI,
                          const int8_t* swp, const int16_t* smp, const int16_t* smh, const int32_t* s, int64_t* sh,
                          int32_t* spart, int32_t R, int32_t SI, int32_t K, void* stream);

/* ... and exact_gemv_g128_experts_qrow_acc (routed experts: exs, epart, ... et, es_out, EN x EK) with
 * exact_gemv_g128_qrow_acc at abits 15 (the shared expert's down GEMV: sxs, spart, ... st, ss_out, SN x SK, R <= 2
 * rows, clearing zero_n int64 of zero) in one launch. No counterpart in the reference, as above. */
int exact_moe_qrow_pair(const int64_t* exs, int64_t eldx, const int32_t* epart, int32_t enparts, const int8_t* ewp,
                        const int16_t* emp, int64_t w_stride, int64_t m_stride, const int32_t* chunk_e,
                        const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks,
                        int32_t chunk, int64_t* et, int32_t* es_out, int32_t EN, int32_t EK, const int64_t* sxs,
                        int64_t sldx, const int32_t* spart, int32_t snparts, const int8_t* swp, const int16_t* smp,
                        const int16_t* smh, int64_t* st, int32_t* ss_out, int32_t R, int32_t SN, int32_t SK,
                        int64_t* zero, int64_t zero_n, void* stream);

/* Combination (moe_exact_kaggle.py:463-467): x[r] += sum_j rs(p_sel[r][j] * rs(t_ed[pidx[r*k+j]], 28 - sh_pair), 20)
 *   + rs(gate[r] * rs(t_sd[r], 28 - sh_s[r]), 16)   (shared expert; skipped if t_sd is NULL).
 * clear_t != 0 leaves t_ed and t_sd zeroed. */
int exact_moe_combine(int64_t* x, int64_t* t_ed, const int32_t* sh_pair, const int64_t* p_sel, const int32_t* pidx,
                      int64_t* t_sd, const int32_t* sh_s, const int64_t* gate, int32_t R, int32_t D, int32_t k,
                      int32_t clear_t, void* stream);

/* ---- model plumbing ------------------------------------------------------------------------------ */
/* x[r] = emb[ids[r]] from an int32 Q16 table (V, D) (exact_llm.py:163; GraphDecoder.step :641). */
int exact_embed(const int32_t* ids, const int32_t* emb, int64_t* x, int32_t R, int32_t D, int32_t V,
                void* stream);

/* Q16 embedding table from a packed int8 table: emb[v][k] = rint(W[v][k] * M[k/128][v] / 2^12)
 * (round half to even, numpy rint), i.e. rint(e * 2^16) of the float row e = W*M/2^28. */
int exact_embed_table(const int8_t* wp, const int16_t* mp, int32_t* emb, int32_t V, int32_t D, void* stream);

/* Logits and greedy tokens: lg = rs(t, 28 - s[r]) (lg may alias t unless clear_t); ids[r] = first argmax
 * of lg[r] (exact_llm.py:180,267). lg or ids may be NULL to skip; clear_t != 0 leaves t zeroed.
 * part: int64 workspace of R * ceil(N / 4096) * 2 (per-slice first maxima). */
int exact_logits_argmax(int64_t* t, const int32_t* s, int64_t* lg, int32_t* ids, int64_t* part, int32_t R,
                        int32_t N, int32_t clear_t, void* stream);

/* exact_logits_argmax with no workspace argument: it allocates nothing (no hipMalloc, hipFree or allocating
 * library call). No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it). The per-slice maxima live in a
 * library-owned device array of 256 KiB per GPU, held until the process ends, so R <= 64 and N <= 2^20
 * (else 2 is returned, nothing launched). The device's array is looked up on the first call on each device,
 * with the stream's device current: make that first call outside a graph capture. Every call on one GPU
 * shares that GPU's array; calls that overlap on one GPU (different streams, or host threads) race. */
int exact_logits_argmax_noalloc(int64_t* t, const int32_t* s, int64_t* lg, int32_t* ids, int32_t R, int32_t N,
                                int32_t clear_t, void* stream);

/* Integer sampler (sample_int, exact_llm.py:256-259) for R logits rows lg (R, V):
 * p = isoftmax_row(rs(lg * tnum, 16)) (Q20), target = (u20 * sum(p)) >> 20 with u20 = splitmix64(seed, step[r]) >> 44,
 * ids[r] = searchsorted(cumsum(p), target, 'right'). tnum = round(2^16 / temperature) (exact_llm.py:249).
 * p_out (optional, R * V) receives p. */
int exact_sample(const int64_t* lg, int32_t R, int32_t V, uint64_t seed, const int32_t* step, int64_t tnum,
                 const int32_t* exp_t, int32_t* ids, int64_t* p_out, void* stream);

/* pos[r] += 1 for r < R (advances a decode step inside a captured graph; GraphDecoder.step :645). */
int exact_advance(int32_t* pos, int32_t R, void* stream);

/* dst[i] = 0 for i < n (graph-safe clear; no hipMemsetAsync). */
int exact_zero(void* dst, int64_t nbytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
