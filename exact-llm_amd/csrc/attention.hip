// q/k/v epilogue with RoPE and KV-cache write, and exact integer attention.
//
// KV cache per layer: kq int16 [B][KV][Smax][hd] (qrow(k, 15) per position, exact_torch.py:147),
// sk int32 [B][KV][Smax] (the per-position shifts), v int64 [B][KV][Smax][hd] (Q16, unquantised,
// SPEC.md:24). Positions beyond pos[r] are never read, which equals the reference's masked static
// cache (speed_fair_kaggle.py:588-589,611: masked slots get probability exactly 0).
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short s2v __attribute__((ext_vector_type(2)));

// a.lo b.lo + a.hi b.hi of two int16 pairs (v_dot2_i32_i16): exact in int32 for |a|, |b| <= 32767
__device__ __forceinline__ int dot2(int a, int b) {
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2v, a), __builtin_bit_cast(s2v, b), 0, false);
}

namespace exact {

// grid (R, H + 2*KV), block 64 (one wave per head slot), hd <= 256
__global__ void k_qkv_rope_cache(int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                 const int64_t* __restrict__ b, const int64_t* __restrict__ cos_t,
                                 const int64_t* __restrict__ sin_t, const int32_t* __restrict__ slot,
                                 const int32_t* __restrict__ pos, int16_t* __restrict__ qq, int32_t* __restrict__ sq,
                                 int16_t* __restrict__ kq, int32_t* __restrict__ sk, int64_t* __restrict__ v, int H,
                                 int KV, int hd, int Smax, int clear_t) {
  __shared__ int64_t y[256];
  const int r = blockIdx.x, hs = blockIdx.y, lane = threadIdx.x;
  const int N = (H + 2 * KV) * hd;
  const int sh = 28 - s[r];
  const int p = pos[r], sl = slot[r];
  if (p < 0 || p >= Smax) return;   // the host keeps positions inside the cache; never write outside it
  const int base = hs * hd;   // q heads, then k heads, then v heads, each hd wide
  for (int j = lane; j < hd; j += 64) {
    const int64_t val = shr64(t[(int64_t)r * N + base + j], sh);
    if (clear_t) t[(int64_t)r * N + base + j] = 0;
    y[j] = b ? val + b[base + j] : val;
  }
  __syncthreads();
  if (hs >= H + KV) {   // v: stored unquantised
    const int kh = hs - H - KV;
    int64_t* dst = v + (((int64_t)sl * KV + kh) * Smax + p) * hd;
    for (int j = lane; j < hd; j += 64) dst[j] = y[j];
    return;
  }
  const int half = hd >> 1;
  int64_t z[4];
  int64_t m = 0;
  int nz = 0;
  for (int j = lane; j < hd; j += 64, ++nz) {
    const int64_t rot = j < half ? -y[j + half] : y[j - half];
    const int64_t val = shr64(y[j] * cos_t[(int64_t)p * hd + j] + rot * sin_t[(int64_t)p * hd + j], EXACT_F);
    z[nz] = val;
    const int64_t a = abs64(val);
    m = a > m ? a : m;
  }
  m = wave_max64(m);
  int q = bitlen64(m) - 15;
  if (q < 0) q = 0;
  nz = 0;
  if (hs < H) {
    int16_t* dst = qq + ((int64_t)r * H + hs) * hd;
    for (int j = lane; j < hd; j += 64, ++nz) {
      int64_t w = shr64(z[nz], q);
      dst[j] = (int16_t)(w > 32767 ? 32767 : (w < -32767 ? -32767 : w));
    }
    if (lane == 0) sq[r * H + hs] = q;
  } else {
    const int kh = hs - H;
    const int64_t row = ((int64_t)sl * KV + kh) * Smax + p;
    int16_t* dst = kq + row * hd;
    for (int j = lane; j < hd; j += 64, ++nz) {
      int64_t w = shr64(z[nz], q);
      dst[j] = (int16_t)(w > 32767 ? 32767 : (w < -32767 ? -32767 : w));
    }
    if (lane == 0) sk[row] = q;
  }
}

// grid (R, H), block ATT_THREADS. Scores in LDS (Smax entries), then max, exp LUT, sum, Q20 p, and p.V:
// thread t owns the dimension pair 2 (t % (hd/2)) and every (ATT_THREADS / (hd/2))-th key, with 16-byte
// V loads, eight in flight.
#ifndef ATT_THREADS
#define ATT_THREADS 512
#endif
#define ATT_KPF 16   // 16-byte key chunks prefetched per thread (hd <= 128)
#ifndef ATT_VPF
#define ATT_VPF 4        // value pairs prefetched per thread (caches of up to ATT_VPF_LONG_S positions)
#endif
#ifndef ATT_VPF_LONG
#define ATT_VPF_LONG 24  // ... and for longer caches (decode at a 256-token context: +3%; at 16 tokens -0.4%)
#endif
#ifndef ATT_VPF_LONG_S
#define ATT_VPF_LONG_S 128
#endif
// long caches whose blocks fit one round: twice the threads per block, so each thread walks half the keys of p.V
#ifndef ATT_WIDE
#define ATT_WIDE 1
#endif
#ifndef ATT_WIDE_THREADS
#define ATT_WIDE_THREADS 1024
#endif
#ifndef ATT_VPF_WIDE
#define ATT_VPF_WIDE 8
#endif
#ifndef ATT_WIDE_BLOCKS
#define ATT_WIDE_BLOCKS 256
#endif
// short caches (at most 2 ATT_THREADS / 8 positions, hd a multiple of 64): 8 threads per cached key for the scores
#ifndef ATT_KS8
#define ATT_KS8 1
#endif
// ... with ATT_WIDE_THREADS-thread blocks for heads of at least ATT_KS8_WIDE_HD dimensions when the (row, head) blocks
// fit one round (7B bs1 decode at a 16-token prompt, A/B: 2.114-2.140 -> 2.101-2.126 ms a step; hd 64 at 0.5B: no gain)
// ... also for caches of ATT_VPF_LONG_S to 2 ATT_WIDE_THREADS / 8 positions (14B bs1 at a 128-token prompt, A/B:
// 4.399-4.434 -> 4.367-4.400 ms a step; 7B at 150 tokens 2.183-2.203 -> 2.170-2.189)
#ifndef ATT_KS8_LONG
#define ATT_KS8_LONG 1
#endif
#ifndef ATT_KS8_LONG4
#define ATT_KS8_LONG4 1
#endif
#ifndef ATT_KS8_WIDE_HD
#define ATT_KS8_WIDE_HD 128
#endif
// ... and value pairs prefetched per thread on the 512-thread short path for heads narrower than ATT_KS8_WIDE_HD
// (0.5B bs1 decode, hd 64: 0.7975-0.7991 -> 0.7940-0.7947 ms a step against 4; 8 on the 1024-thread path: 7B +5 us)
#ifndef ATT_VPF_NARROW
#define ATT_VPF_NARROW 8
#endif
// most blocks per (row, head) that exact_attention_qkv_split gives the p.V of a short cache
#ifndef ATT_DS
#define ATT_DS 4
#endif
// launches whose (row, head) blocks run in several rounds (batched decode): the 8-threads-per-key path up to
// 4 ATT_THREADS / 8 cached positions (14B bs8 at a 135-token context, warm caches: 19.6 -> 11.5 us, against 13.7 us
// for exact_qkv_rope_cache + exact_attention), the exp table read from global memory (ATT_MR_GT; cold caches, 48
// layers' KV in turn: 17.0 us against 25.6 with the table staged into LDS) and ATT_MR_VPF value pairs prefetched
// (cold: 4 18.1 us, 8 17.0, 12 22.8, 16 20.6; 14B bs8 decode 5.32-5.33 -> 5.27-5.29 ms a step with 8 against 4)
#ifndef ATT_KS8_MR
#define ATT_KS8_MR 1
#endif
// ... and for the one-round launches split 4 ways (7B bs1 1.988 -> 1.978 ms a step, MoE 1.756 -> 1.740, 0.5B +0.5%)
#ifndef ATT_GT1
#define ATT_GT1 1
#endif
#ifndef ATT_MR_VPF
#define ATT_MR_VPF 8
#endif
#ifndef ATT_GQA
#define ATT_GQA 1
#endif
#ifndef ATT_GQA_NT
#define ATT_GQA_NT 512
#endif
// ... for caches longer than this (14B bs8, cold caches of 48 layers in turn: at 256 positions 23.2 against 25.1 us
// a launch, at 148 positions 18.8 against 17.1, decode 5.37 against 5.28 ms a step; 1024-thread blocks: slower still)
#ifndef ATT_GQA_MIN_S
#define ATT_GQA_MIN_S 192
#endif
#ifndef ATT_MR_GT
#define ATT_MR_GT 1
#endif
#ifndef ATT_VPF_LONG_BLOCKS
#define ATT_VPF_LONG_BLOCKS 256
#endif
// PRE: prefetch the first key and VPF value pairs with the query (one round of blocks: the registers they take
// cost more occupancy than they save latency when the blocks run in several rounds)
template <int VPF, bool PRE>
__global__ __launch_bounds__(ATT_THREADS) void k_attention(const int16_t* __restrict__ qq, const int32_t* __restrict__ sq,
                                                           const int16_t* __restrict__ kq, const int32_t* __restrict__ sk,
                                                           const int64_t* __restrict__ v, const int32_t* __restrict__ slot,
                                                           const int32_t* __restrict__ pos, const int32_t* __restrict__ expt,
                                                           int64_t* __restrict__ out, int32_t* __restrict__ obits, int H,
                                                           int KV, int hd, int Smax, int INV) {
  extern __shared__ int64_t sc[];   // Smax entries
  __shared__ int32_t qs[256];
  __shared__ int ored[ATT_THREADS / 64];
  __shared__ int64_t red[16];
  __shared__ int64_t part[ATT_THREADS * 2];
  const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int kh = h / (H / KV);
  const int S = min(pos[r] + 1, Smax), sl = slot[r];
  const int sqv = sq[r * H + h];
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  const int npair = hd >> 1, nparts = blockDim.x / npair;   // hd divides 2 * ATT_THREADS
  const int dp = tid % npair, pp = tid / npair;
  // loads that do not depend on the query, issued with it: this thread's first key and its first VPF value pairs
  v4i kpre[ATT_KPF];
  int skpre = 0;
  const bool kp = PRE && hd <= 8 * ATT_KPF && tid < S;
  if (kp) {
    const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + tid) * hd);
#pragma unroll
    for (int j8 = 0; j8 < ATT_KPF; ++j8)
      if (j8 < hd / 8) kpre[j8] = kr[j8];
    skpre = sk[cbase + tid];
  }
  v4i vpre[VPF];
  const int64_t* vb = v + cbase * hd + 2 * dp;
  if constexpr (PRE) {
#pragma unroll
    for (int i = 0; i < VPF; ++i) {
      const int si = pp + i * nparts;
      if (pp < nparts && si < S) vpre[i] = *reinterpret_cast<const v4i*>(vb + (int64_t)si * hd);
    }
  }
  for (int j = tid; j < hd; j += blockDim.x) qs[j] = qq[((int64_t)r * H + h) * hd + j];
  __syncthreads();
  int64_t mx = INT64_MIN;
  for (int si = tid; si < S; si += blockDim.x) {
    // 16-byte key loads, four in flight; each pair of int16 products is exact in int32 (< 2^31)
    const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + si) * hd);
    int64_t dot = 0;
    int skv;
    if (kp && si == tid) {   // the prefetched first key
#pragma unroll
      for (int j8 = 0; j8 < ATT_KPF; ++j8) {
        if (j8 < hd / 8) {
          const v4i kk = kpre[j8];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int j = j8 * 8 + 2 * c;
            dot += (int64_t)(qs[j] * (int32_t)(int16_t)(kk[c] & 0xffff) + qs[j + 1] * (int32_t)(int16_t)(kk[c] >> 16));
          }
        }
      }
      skv = skpre;
    } else {
#pragma unroll 4
      for (int j8 = 0; j8 < hd / 8; ++j8) {
        const v4i kk = kr[j8];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int j = j8 * 8 + 2 * c;
          dot += (int64_t)(qs[j] * (int32_t)(int16_t)(kk[c] & 0xffff) + qs[j + 1] * (int32_t)(int16_t)(kk[c] >> 16));
        }
      }
      skv = sk[cbase + si];
    }
    const int64_t val = shr64(dot * INV, 32 - sqv - skv);
    sc[si] = val;
    mx = val > mx ? val : mx;
  }
  mx = block_max64(mx, red);
  int64_t es = 0;
  for (int si = tid; si < S; si += blockDim.x) {
    const int64_t e = lut_exp(expt, mx - sc[si]);
    sc[si] = e;
    es += e;
  }
  es = block_sum64(es, red);
  for (int si = tid; si < S; si += blockDim.x) sc[si] = floordiv_pos(shl64(sc[si], 20), es);
  __syncthreads();
  int64_t a0 = 0, a1 = 0;
  if (pp < nparts) {
#pragma unroll
    for (int i = 0; i < (PRE ? VPF : 0); ++i) {
      const int si = pp + i * nparts;
      if (si < S) {
        const v4i vv = vpre[i];
        const int64_t p = sc[si];
        a0 = (int64_t)((uint64_t)a0 + (uint64_t)(p * (((int64_t)vv[1] << 32) | (uint32_t)vv[0])));
        a1 = (int64_t)((uint64_t)a1 + (uint64_t)(p * (((int64_t)vv[3] << 32) | (uint32_t)vv[2])));
      }
    }
#pragma unroll 8
    for (int si = pp + (PRE ? VPF : 0) * nparts; si < S; si += nparts) {
      const v4i vv = *reinterpret_cast<const v4i*>(vb + (int64_t)si * hd);
      const int64_t p = sc[si];
      a0 = (int64_t)((uint64_t)a0 + (uint64_t)(p * (((int64_t)vv[1] << 32) | (uint32_t)vv[0])));
      a1 = (int64_t)((uint64_t)a1 + (uint64_t)(p * (((int64_t)vv[3] << 32) | (uint32_t)vv[2])));
    }
  }
  part[2 * tid] = a0;
  part[2 * tid + 1] = a1;
  __syncthreads();
  int m = 0;
  if (tid < hd) {
    const int d = tid;   // dimension d sits in pair d / 2, half d % 2
    uint64_t tot = 0;
    for (int k = 0; k < nparts; ++k) tot += (uint64_t)part[2 * (k * npair + (d >> 1)) + (d & 1)];
    const int64_t o = shr64((int64_t)tot, 20);
    out[((int64_t)r * H + h) * hd + d] = o;
    m = bitlen64(abs64(o));
  }
  if (obits) {   // bit length of this head's max |out|, for the row quantisation of the o-projection input
    m = block_max_i32(m, ored);
    if (tid == 0) obits[(int64_t)r * H + h] = m;
  }
}

// Decode rows that each own their (slot, position) (one row, or rows of different sequences): the q/k/v epilogue,
// RoPE and cache write of k_qkv_rope_cache and the attention of k_attention in one launch. Block (r, h) rebuilds
// its query head and its KV head's new key and value at pos[r] from the totals t, attends over the cached
// positions < pos[r] and over the new one from LDS, and the first query head of each KV group writes the new key
// and value into the cache (the other blocks never read that position from the cache). The arithmetic is the
// two kernels' own: the same shifts, rounding, RoPE, quantisation and dot products. t is left as it is.
// Latency: everything that does not depend on the new token (the RoPE row, each thread's first cached key and
// its first ATT_VPF value pairs) is loaded together with t, so the block waits on memory about once before the
// exp table.
// KPF: 16-byte chunks of each thread's first cached key loaded with the totals (0: none).
// KS = 8 (caches of at most KP NT / 8 positions, hd a multiple of 64): the scores of the cached keys are computed by 8
// threads per key, hd / 8 dimensions each (coalesced 16-byte loads of the key row, a sum over the 8 lanes), NT / 8 keys
// per pass and at most KP passes, all loaded with the totals; KPF is then unused.
// DS > 1: DS blocks per (row, head) (blockIdx.z = slice), each with the whole softmax and the p.V of hd / DS
// dimensions, so each thread's share of the value rows is loaded with the keys, at the start; needs hd / (2 DS) a
// power of two of at most 64. obits gets obn (a multiple of DS) entries per head, each block the max of its slice.
// GT: exp table lookups from global memory (cached), not staged into LDS: 41 KiB less LDS a block, for launches whose
// blocks run in several rounds
template <int VPF, int NT = ATT_THREADS, int KPF = ATT_KPF, int KS = 1, int KP = 2, int DS = 1, bool GT = false>
__global__ __launch_bounds__(NT) void k_attention_qkv(const int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                                               const int64_t* __restrict__ b, const int64_t* __restrict__ cos_t,
                                                               const int64_t* __restrict__ sin_t, const int32_t* __restrict__ slot,
                                                               const int32_t* __restrict__ pos, int16_t* __restrict__ kq,
                                                               int32_t* __restrict__ sk, int64_t* __restrict__ v,
                                                               const int32_t* __restrict__ expt, int64_t* __restrict__ out,
                                                               int32_t* __restrict__ obits, int H, int KV, int hd, int Smax,
                                                               int INV, int obn) {
  extern __shared__ int64_t sc[];   // Smax entries
  __shared__ int64_t y[3][256];     // q head, new key, new value: shr(t, 28 - s) + b
  __shared__ int32_t qs[256], kn[256];
  __shared__ __attribute__((aligned(16))) int16_t qs16[256];   // the query head again as int16, pairs for v_dot2
  __shared__ __attribute__((aligned(16))) int32_t texp[EXACT_EXP_N + 2];
  __shared__ int32_t shq[2];
  __shared__ int ored[16];
  __shared__ int64_t red[16], red2[16];
  __shared__ int64_t part[NT * 2];
  const int r = blockIdx.x, h = blockIdx.y, ds = DS > 1 ? (int)blockIdx.z : 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = H / KV, kh = h / grp;
  const int N = (H + 2 * KV) * hd;
  const int p = pos[r], sl = slot[r];
  const int hds = hd / DS;   // this block's output dimensions [ds hds, (ds + 1) hds)
  if (p < 0 || p >= Smax) {   // the host keeps positions inside the cache; write nothing there
    for (int d = tid; d < hds; d += blockDim.x) out[((int64_t)r * H + h) * hd + ds * hds + d] = 0;
    if (obits && tid < obn / DS) obits[((int64_t)r * H + h) * obn + ds * (obn / DS) + tid] = 0;
    return;
  }
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  const int npair = hds >> 1, nparts = blockDim.x / npair;   // value pairs of the slice, threads per pair
  const int dp = ds * npair + tid % npair, pp = tid / npair;
  // ---- loads that do not depend on the new token, issued with the totals
  v4i kpre[KPF > 0 && KS == 1 ? KPF : 1];
  int skpre = 0;
  // KS = 8: thread (key kg = tid / 8, lane kl = tid % 8) holds dims [kl hd / 8, (kl + 1) hd / 8) of keys kg,
  // kg + NT / 8, ... (KP passes), at most 4 chunks of 16 bytes each
  constexpr int NVC = KP > 2 ? 2 : 4;   // chunks a thread holds per key (the 4-pass variant runs at hd 128 only)
  v4i ks8[KP][NVC];
  int sks8[KP];
#pragma unroll
  for (int ps = 0; ps < KP; ++ps) sks8[ps] = 0;
  const int kg = tid >> 3, kl = tid & 7;
  if constexpr (KS == 8) {
    const int nv = hd >> 6;   // 16-byte chunks per thread and key
#pragma unroll
    for (int ps = 0; ps < KP; ++ps) {
      const int si = kg + ps * (NT / 8);
      if (si < p) {
        const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + si) * hd + kl * (hd >> 3));
#pragma unroll
        for (int c = 0; c < NVC; ++c)
          if (c < nv) ks8[ps][c] = kr[c];
        sks8[ps] = sk[cbase + si];
      }
    }
  }
  const bool kp = KS == 1 && KPF > 0 && hd <= 8 * KPF && tid < p;
  if (kp) {
    const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + tid) * hd);
#pragma unroll
    for (int j8 = 0; j8 < KPF; ++j8)
      if (j8 < hd / 8) kpre[j8] = kr[j8];
    skpre = sk[cbase + tid];
  }
  v4i vpre[VPF];
  const int64_t* vb = v + cbase * hd + 2 * dp;
#pragma unroll
  for (int i = 0; i < VPF; ++i) {
    const int si = pp + i * nparts;
    if (pp < nparts && si < p) vpre[i] = *reinterpret_cast<const v4i*>(vb + (int64_t)si * hd);
  }
  int64_t cs[4][2];
  if (wave < 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = lane + 64 * i;
      cs[i][0] = j < hd ? cos_t[(int64_t)p * hd + j] : 0;
      cs[i][1] = j < hd ? sin_t[(int64_t)p * hd + j] : 0;
    }
  }
  // the new token's totals (and biases) for the query head, the new key and the new value, loaded before the exp
  // table's LDS stores, which wait for the table's loads: issued after them, these would wait a round trip more
  constexpr int TV = (3 * 256 + NT - 1) / NT;   // hd <= 256
  int64_t tv[TV], bv[TV];
#pragma unroll
  for (int i = 0; i < TV; ++i) {
    const int j = tid + i * NT;
    tv[i] = bv[i] = 0;
    if (j < 3 * hd) {
      const int which = j / hd, jj = j - which * hd;
      const int base = which == 0 ? h * hd : (which == 1 ? (H + kh) * hd : (H + KV + kh) * hd);
      tv[i] = t[(int64_t)r * N + base + jj];
      if (b) bv[i] = b[base + jj];
    }
  }
  const int sh = 28 - s[r];
  if constexpr (!GT) {   // the exp table into LDS: every piece loaded before the first store, with the loads above
    constexpr int NV = EXACT_EXP_N / 4, NK = (NV + NT - 1) / NT;
    v4i te[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k)
      if (tid + k * NT < NV) te[k] = reinterpret_cast<const v4i*>(expt)[tid + k * NT];
    const int tail = tid < EXACT_EXP_N - 4 * NV ? expt[4 * NV + tid] : 0;
#pragma unroll
    for (int k = 0; k < NK; ++k)
      if (tid + k * NT < NV) reinterpret_cast<v4i*>(texp)[tid + k * NT] = te[k];
    if (tid < EXACT_EXP_N - 4 * NV) texp[4 * NV + tid] = tail;
  }
#pragma unroll
  for (int i = 0; i < TV; ++i) {
    const int j = tid + i * NT;
    if (j < 3 * hd) {
      const int which = j / hd, jj = j - which * hd;
      y[which][jj] = shr64(tv[i], sh) + bv[i];
    }
  }
  __syncthreads();
  if (wave < 2) {   // wave 0: RoPE + qrow of the query head, wave 1: of the new key (k_qkv_rope_cache's steps)
    const int half = hd >> 1;
    const int64_t* yy = y[wave];
    int64_t z[4];
    int64_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = lane + 64 * i;
      z[i] = 0;
      if (j < hd) {
        const int64_t rot = j < half ? -yy[j + half] : yy[j - half];
        z[i] = shr64(yy[j] * cs[i][0] + rot * cs[i][1], EXACT_F);
        const int64_t a = abs64(z[i]);
        m = a > m ? a : m;
      }
    }
    m = wave_max64(m);
    int q = bitlen64(m) - 15;
    if (q < 0) q = 0;
    int32_t* dst = wave == 0 ? qs : kn;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = lane + 64 * i;
      if (j < hd) {
        const int64_t w = shr64(z[i], q);
        dst[j] = (int32_t)(w > 32767 ? 32767 : (w < -32767 ? -32767 : w));
        if (wave == 0) qs16[j] = (int16_t)dst[j];
      }
    }
    if (lane == 0) shq[wave] = q;
  }
  __syncthreads();
  const int sqv = shq[0], skn = shq[1];
  if (h % grp == 0 && ds == 0) {   // one block per KV head writes the new position
    for (int j = tid; j < hd; j += blockDim.x) {
      kq[(cbase + p) * hd + j] = (int16_t)kn[j];
      v[(cbase + p) * hd + j] = y[2][j];
    }
    if (tid == 0) sk[cbase + p] = skn;
  }
  const int S = p + 1;
  int64_t mx = INT64_MIN;
  if constexpr (KS == 8) {
    const int nv = hd >> 6;
#pragma unroll
    for (int ps = 0; ps < KP; ++ps) {
      const int si = kg + ps * (NT / 8);
      int64_t dot = 0;
      if (si < p) {
#pragma unroll
        for (int c = 0; c < NVC; ++c) {
          if (c < nv) {
            const v4i kk = ks8[ps][c], qq = reinterpret_cast<const v4i*>(qs16 + kl * (hd >> 3))[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) dot += (int64_t)dot2(qq[e], kk[e]);
          }
        }
      }
      // sum over the 8 lanes of the key (lanes 8 kg .. 8 kg + 7): exchange with lane ^ 1, lane ^ 2, then the mirrored
      // lane of the 8-lane half row; every lane of the key ends with its dot product
      dot += dpp64<0xB1>(dot);
      dot += dpp64<0x4E>(dot);
      dot += dpp64<0x141>(dot);
      if (si < p) {
        const int64_t val = shr64(dot * INV, 32 - sqv - sks8[ps]);
        if (kl == 0) sc[si] = val;
        mx = val > mx ? val : mx;
      }
    }
  }
  for (int si = tid; KS == 1 && si < p; si += blockDim.x) {
    const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + si) * hd);
    int64_t dot = 0;
    int skv;
    if (kp && si == tid) {   // the prefetched first key
#pragma unroll
      for (int j8 = 0; j8 < KPF; ++j8) {
        if (j8 < hd / 8) {
          const v4i kk = kpre[j8], qq = reinterpret_cast<const v4i*>(qs16)[j8];
#pragma unroll
          for (int c = 0; c < 4; ++c) dot += (int64_t)dot2(qq[c], kk[c]);
        }
      }
      skv = skpre;
    } else {
#pragma unroll 4
      for (int j8 = 0; j8 < hd / 8; ++j8) {
        const v4i kk = kr[j8], qq = reinterpret_cast<const v4i*>(qs16)[j8];
#pragma unroll
        for (int c = 0; c < 4; ++c) dot += (int64_t)dot2(qq[c], kk[c]);
      }
      skv = sk[cbase + si];
    }
    const int64_t val = shr64(dot * INV, 32 - sqv - skv);
    sc[si] = val;
    mx = val > mx ? val : mx;
  }
  if (wave == (int)(p % blockDim.x) >> 6) {   // the new key, from LDS: the wave of thread p % blockDim.x, lanes over dims
    int64_t psum = 0;
    for (int j = lane; j < hd; j += 64) psum += (int64_t)qs[j] * kn[j];   // exact: |q k| < 2^30, 256 of them
    const int64_t dot = wave_sum64(psum);
    if (tid == (int)(p % blockDim.x)) {   // that thread owns sc[p] in the loops below
      const int64_t val = shr64(dot * INV, 32 - sqv - skn);
      sc[p] = val;
      mx = val > mx ? val : mx;
    }
  }
  mx = block_max64_1(mx, red);
  int64_t es = 0;
  for (int si = tid; si < S; si += blockDim.x) {
    const int64_t e = lut_exp(GT ? expt : texp, mx - sc[si]);
    sc[si] = e;
    es += e;
  }
  es = block_sum64_1(es, red2);
  const double res = 1.0 / (double)es;   // one reciprocal; each quotient estimate is corrected exactly
  for (int si = tid; si < S; si += blockDim.x) sc[si] = floordiv_rcp(shl64(sc[si], 20), es, res);
  __syncthreads();
  int64_t a0 = 0, a1 = 0;
  if (pp < nparts) {
#pragma unroll
    for (int i = 0; i < VPF; ++i) {
      const int si = pp + i * nparts;
      if (si < p) {
        const v4i vv = vpre[i];
        const int64_t pr = sc[si];
        a0 = (int64_t)((uint64_t)a0 + (uint64_t)(pr * (((int64_t)vv[1] << 32) | (uint32_t)vv[0])));
        a1 = (int64_t)((uint64_t)a1 + (uint64_t)(pr * (((int64_t)vv[3] << 32) | (uint32_t)vv[2])));
      }
    }
#pragma unroll 8
    for (int si = pp + VPF * nparts; si < p; si += nparts) {
      const v4i vv = *reinterpret_cast<const v4i*>(vb + (int64_t)si * hd);
      const int64_t pr = sc[si];
      a0 = (int64_t)((uint64_t)a0 + (uint64_t)(pr * (((int64_t)vv[1] << 32) | (uint32_t)vv[0])));
      a1 = (int64_t)((uint64_t)a1 + (uint64_t)(pr * (((int64_t)vv[3] << 32) | (uint32_t)vv[2])));
    }
    if (pp == p % nparts) {   // the new value, from LDS
      const int64_t pr = sc[p];
      a0 = (int64_t)((uint64_t)a0 + (uint64_t)(pr * y[2][2 * dp]));
      a1 = (int64_t)((uint64_t)a1 + (uint64_t)(pr * y[2][2 * dp + 1]));
    }
  }
  int m = 0;
  if constexpr (DS == 1) {
    part[2 * tid] = a0;
    part[2 * tid + 1] = a1;
    __syncthreads();
    if (tid < hd) {
      const int d = tid;
      uint64_t tot = 0;
      for (int k = 0; k < nparts; ++k) tot += (uint64_t)part[2 * (k * npair + (d >> 1)) + (d & 1)];
      const int64_t o = shr64((int64_t)tot, 20);
      out[((int64_t)r * H + h) * hd + d] = o;
      m = bitlen64(abs64(o));
    }
  } else {
    // lanes l, l ^ npair, l ^ 2 npair ... of a wave hold the same pair: fold them (sums modulo 2^64), then the waves
    for (int o = npair; o < 64; o <<= 1) {
      a0 = (int64_t)((uint64_t)a0 + (uint64_t)__shfl_xor((long long)a0, o));
      a1 = (int64_t)((uint64_t)a1 + (uint64_t)__shfl_xor((long long)a1, o));
    }
    if (lane < npair) {
      part[wave * hds + 2 * lane] = a0;
      part[wave * hds + 2 * lane + 1] = a1;
    }
    __syncthreads();
    if (tid < hds) {
      uint64_t tot = 0;
#pragma unroll
      for (int w = 0; w < NT / 64; ++w) tot += (uint64_t)part[w * hds + tid];
      const int64_t o = shr64((int64_t)tot, 20);
      out[((int64_t)r * H + h) * hd + ds * hds + tid] = o;
      m = bitlen64(abs64(o));
    }
  }
  if (obits) {
    m = block_max_i32(m, ored);
    if (tid < obn / DS) obits[((int64_t)r * H + h) * obn + ds * (obn / DS) + tid] = m;
  }
}

// Batched decode whose (row, head) blocks would take several rounds: one block per (row r, KV head kh, dimension slice
// ds) for all HB = H / KV query heads of the group, so the group's cached keys and values are loaded once. The
// arithmetic per head is k_attention_qkv's (8 threads per cached key, exp table read from global memory, the p.V of
// hd / DS dimensions): the same shifts, rounding, RoPE, quantisation, products and sums, so the results are equal.
// hd <= 128 (a multiple of 64); caches of at most KP NT / 8 positions; hd / (2 DS) a power of two of at most 64.
template <int VPF, int NT, int KP, int DS, int HB>
__global__ __launch_bounds__(NT) void k_attention_gqa(const int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                                      const int64_t* __restrict__ b, const int64_t* __restrict__ cos_t,
                                                      const int64_t* __restrict__ sin_t, const int32_t* __restrict__ slot,
                                                      const int32_t* __restrict__ pos, int16_t* __restrict__ kq,
                                                      int32_t* __restrict__ sk, int64_t* __restrict__ v,
                                                      const int32_t* __restrict__ expt, int64_t* __restrict__ out,
                                                      int32_t* __restrict__ obits, int H, int KV, int hd, int Smax, int INV,
                                                      int obn) {
  constexpr int NW = NT / 64;
  extern __shared__ int64_t sc[];   // HB x Smax scores, then exponentials, then probabilities
  __shared__ int64_t y[HB + 2][128];   // the group's query heads, the new key, the new value: shr(t, 28 - s) + b
  __shared__ int32_t kn[128];
  __shared__ __attribute__((aligned(16))) int16_t qs16[HB][128];
  __shared__ int32_t shq[HB + 1];
  __shared__ int64_t red[NW][HB], red2[NW][HB];
  __shared__ int64_t part[NW][HB][128 / DS];
  __shared__ int bl[HB][128 / DS];
  const int r = blockIdx.x, kh = blockIdx.y, ds = DS > 1 ? (int)blockIdx.z : 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h0 = kh * HB;
  const int N = (H + 2 * KV) * hd;
  const int p = pos[r], sl = slot[r];
  const int hds = hd / DS;
  if (p < 0 || p >= Smax) {   // the host keeps positions inside the cache; write nothing there
    for (int i = tid; i < HB * hds; i += NT) out[((int64_t)r * H + h0 + i / hds) * hd + ds * hds + i % hds] = 0;
    if (obits && tid < HB * (obn / DS))
      obits[((int64_t)r * H + h0 + tid / (obn / DS)) * obn + ds * (obn / DS) + tid % (obn / DS)] = 0;
    return;
  }
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  const int npair = hds >> 1, nparts = NT / npair;
  const int dp = ds * npair + tid % npair, pp = tid / npair;
  // keys: thread (kg = tid / 8, kl = tid % 8) holds dims [kl hd / 8, (kl + 1) hd / 8) of keys kg, kg + NT / 8, ...
  v4i ks8[KP][2];
  int sks8[KP];
  const int kg = tid >> 3, kl = tid & 7, nv = hd >> 6;
#pragma unroll
  for (int ps = 0; ps < KP; ++ps) {
    sks8[ps] = 0;
    const int si = kg + ps * (NT / 8);
    if (si < p) {
      const v4i* kr = reinterpret_cast<const v4i*>(kq + (cbase + si) * hd + kl * (hd >> 3));
#pragma unroll
      for (int c = 0; c < 2; ++c)
        if (c < nv) ks8[ps][c] = kr[c];
      sks8[ps] = sk[cbase + si];
    }
  }
  v4i vpre[VPF];
  const int64_t* vb = v + cbase * hd + 2 * dp;
#pragma unroll
  for (int i = 0; i < VPF; ++i) {
    const int si = pp + i * nparts;
    if (si < p) vpre[i] = *reinterpret_cast<const v4i*>(vb + (int64_t)si * hd);
  }
  int64_t cs[2][2];
  if (wave <= HB) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = lane + 64 * i;
      cs[i][0] = j < hd ? cos_t[(int64_t)p * hd + j] : 0;
      cs[i][1] = j < hd ? sin_t[(int64_t)p * hd + j] : 0;
    }
  }
  constexpr int TV = ((HB + 2) * 128 + NT - 1) / NT;
  int64_t tv[TV], bv[TV];
#pragma unroll
  for (int i = 0; i < TV; ++i) {
    const int j = tid + i * NT;
    tv[i] = bv[i] = 0;
    if (j < (HB + 2) * hd) {
      const int which = j / hd, jj = j - which * hd;
      const int base = which < HB ? (h0 + which) * hd : (which == HB ? (H + kh) * hd : (H + KV + kh) * hd);
      tv[i] = t[(int64_t)r * N + base + jj];
      if (b) bv[i] = b[base + jj];
    }
  }
  const int sh = 28 - s[r];
#pragma unroll
  for (int i = 0; i < TV; ++i) {
    const int j = tid + i * NT;
    if (j < (HB + 2) * hd) {
      const int which = j / hd, jj = j - which * hd;
      y[which][jj] = shr64(tv[i], sh) + bv[i];
    }
  }
  __syncthreads();
  if (wave <= HB) {   // waves 0 .. HB - 1: RoPE + qrow of the query heads, wave HB: of the new key
    const int half = hd >> 1;
    const int64_t* yy = y[wave];
    int64_t z[2];
    int64_t m = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = lane + 64 * i;
      z[i] = 0;
      if (j < hd) {
        const int64_t rot = j < half ? -yy[j + half] : yy[j - half];
        z[i] = shr64(yy[j] * cs[i][0] + rot * cs[i][1], EXACT_F);
        const int64_t a = abs64(z[i]);
        m = a > m ? a : m;
      }
    }
    m = wave_max64(m);
    int q = bitlen64(m) - 15;
    if (q < 0) q = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = lane + 64 * i;
      if (j < hd) {
        const int64_t w = shr64(z[i], q);
        const int32_t wc = (int32_t)(w > 32767 ? 32767 : (w < -32767 ? -32767 : w));
        if (wave < HB) qs16[wave][j] = (int16_t)wc;
        else kn[j] = wc;
      }
    }
    if (lane == 0) shq[wave] = q;
  }
  __syncthreads();
  const int skn = shq[HB];
  if (ds == 0) {   // one block per (row, KV head) writes the new position
    for (int j = tid; j < hd; j += NT) {
      kq[(cbase + p) * hd + j] = (int16_t)kn[j];
      v[(cbase + p) * hd + j] = y[HB + 1][j];
    }
    if (tid == 0) sk[cbase + p] = skn;
  }
  const int S = p + 1;
  int64_t mx[HB];
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) mx[hb] = INT64_MIN;
#pragma unroll
  for (int ps = 0; ps < KP; ++ps) {
    const int si = kg + ps * (NT / 8);
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      int64_t dot = 0;
      if (si < p) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          if (c < nv) {
            const v4i kk = ks8[ps][c], qq = reinterpret_cast<const v4i*>(qs16[hb] + kl * (hd >> 3))[c];
#pragma unroll
            for (int e = 0; e < 4; ++e) dot += (int64_t)dot2(qq[e], kk[e]);
          }
        }
      }
      dot += dpp64<0xB1>(dot);
      dot += dpp64<0x4E>(dot);
      dot += dpp64<0x141>(dot);
      if (si < p) {
        const int64_t val = shr64(dot * INV, 32 - shq[hb] - sks8[ps]);
        if (kl == 0) sc[hb * Smax + si] = val;
        mx[hb] = val > mx[hb] ? val : mx[hb];
      }
    }
  }
  if (wave == (int)(p % NT) >> 6) {   // the new key, from LDS: the wave of thread p % NT, lanes over dims
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      int64_t psum = 0;
      for (int j = lane; j < hd; j += 64) psum += (int64_t)qs16[hb][j] * kn[j];
      const int64_t dot = wave_sum64(psum);
      if (tid == (int)(p % NT)) {   // that thread owns sc[hb][p] in the loops below
        const int64_t val = shr64(dot * INV, 32 - shq[hb] - skn);
        sc[hb * Smax + p] = val;
        mx[hb] = val > mx[hb] ? val : mx[hb];
      }
    }
  }
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int64_t m = wave_max64(mx[hb]);
    if (lane == 0) red[wave][hb] = m;
  }
  __syncthreads();
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    int64_t m = red[0][hb];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = red[w][hb] > m ? red[w][hb] : m;
    mx[hb] = m;
  }
  int64_t es[HB];
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) es[hb] = 0;
  for (int si = tid; si < S; si += NT) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int64_t e = lut_exp(expt, mx[hb] - sc[hb * Smax + si]);
      sc[hb * Smax + si] = e;
      es[hb] += e;
    }
  }
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    const int64_t e = wave_sum64(es[hb]);
    if (lane == 0) red2[wave][hb] = e;
  }
  __syncthreads();
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    uint64_t e = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) e += (uint64_t)red2[w][hb];
    es[hb] = (int64_t)e;
  }
  for (int si = tid; si < S; si += NT) {
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const double res = 1.0 / (double)es[hb];   // one reciprocal per head; each quotient estimate is corrected exactly
      sc[hb * Smax + si] = floordiv_rcp(shl64(sc[hb * Smax + si], 20), es[hb], res);
    }
  }
  __syncthreads();
  int64_t a0[HB], a1[HB];
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) a0[hb] = a1[hb] = 0;
  auto madd = [&](const v4i vv, int si) {
    const int64_t lo = ((int64_t)vv[1] << 32) | (uint32_t)vv[0], hi = ((int64_t)vv[3] << 32) | (uint32_t)vv[2];
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int64_t pr = sc[hb * Smax + si];
      a0[hb] = (int64_t)((uint64_t)a0[hb] + (uint64_t)(pr * lo));
      a1[hb] = (int64_t)((uint64_t)a1[hb] + (uint64_t)(pr * hi));
    }
  };
#pragma unroll
  for (int i = 0; i < VPF; ++i) {
    const int si = pp + i * nparts;
    if (si < p) madd(vpre[i], si);
  }
  for (int si = pp + VPF * nparts; si < p; si += nparts) madd(*reinterpret_cast<const v4i*>(vb + (int64_t)si * hd), si);
  if (pp == p % nparts) {   // the new value, from LDS
#pragma unroll
    for (int hb = 0; hb < HB; ++hb) {
      const int64_t pr = sc[hb * Smax + p];
      a0[hb] = (int64_t)((uint64_t)a0[hb] + (uint64_t)(pr * y[HB + 1][2 * dp]));
      a1[hb] = (int64_t)((uint64_t)a1[hb] + (uint64_t)(pr * y[HB + 1][2 * dp + 1]));
    }
  }
  // lanes l, l ^ npair, ... of a wave hold the same pair: fold them (sums modulo 2^64), then the waves
#pragma unroll
  for (int hb = 0; hb < HB; ++hb) {
    for (int o = npair; o < 64; o <<= 1) {
      a0[hb] = (int64_t)((uint64_t)a0[hb] + (uint64_t)__shfl_xor((long long)a0[hb], o));
      a1[hb] = (int64_t)((uint64_t)a1[hb] + (uint64_t)__shfl_xor((long long)a1[hb], o));
    }
    if (lane < npair) {
      part[wave][hb][2 * lane] = a0[hb];
      part[wave][hb][2 * lane + 1] = a1[hb];
    }
  }
  __syncthreads();
  for (int i = tid; i < HB * hds; i += NT) {
    const int hb = i / hds, dl = i - hb * hds;
    uint64_t tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += (uint64_t)part[w][hb][dl];
    const int64_t o = shr64((int64_t)tot, 20);
    out[((int64_t)r * H + h0 + hb) * hd + ds * hds + dl] = o;
    bl[hb][dl] = bitlen64(abs64(o));
  }
  if (obits) {
    __syncthreads();
    if (tid < HB) {
      int m = 0;
      for (int dl = 0; dl < hds; ++dl) m = bl[tid][dl] > m ? bl[tid][dl] : m;
      for (int i = 0; i < obn / DS; ++i) obits[((int64_t)r * H + h0 + tid) * obn + ds * (obn / DS) + i] = m;
    }
  }
}

}  // namespace exact

using namespace exact;

// one launch of a k_attention_qkv variant; the scores take Smax * 8 bytes of LDS, up to 64 KiB beside the static arrays
template <int VPF, int NT, int KPF = ATT_KPF, int KS = 1, int KP = 2, int DS = 1, bool GT = false>
static void att_qkv_go(int R, int H, size_t lds, hipStream_t st, const int64_t* t, const int32_t* s, const int64_t* b,
                       const int64_t* cos_t, const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq,
                       int32_t* sk, int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int KV, int hd, int Smax,
                       int INV, int obn) {
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_attention_qkv<VPF, NT, KPF, KS, KP, DS, GT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 8192 * 8);
    attr_set = true;
  }
  hipLaunchKernelGGL((k_attention_qkv<VPF, NT, KPF, KS, KP, DS, GT>), dim3(R, H, DS), dim3(NT), lds, st, t, s, b, cos_t, sin_t,
                     slot, pos, kq, sk, v, exp_t, out, obits, H, KV, hd, Smax, INV, obn);
}

// one k_attention_gqa launch: dimension slices ds (4, 2 or 1) of the (row, KV head) blocks
template <int DS, int HB>
static void att_gqa_go1(int R, int H, size_t, hipStream_t st, const int64_t* t, const int32_t* s, const int64_t* b,
                        const int64_t* cos_t, const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq,
                        int32_t* sk, int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int KV, int hd, int Smax,
                        int INV, int obn) {
  constexpr int NT = ATT_GQA_NT, KP = 2048 / NT;       // 256 cached positions in KP passes of NT / 8 keys
  constexpr int NP = NT * 2 * DS / 128;                 // threads per value pair at hd 128
  constexpr int VPF = (256 + NP - 1) / NP < 16 ? (256 + NP - 1) / NP : 16;
  static bool attr_set = false;
  const size_t lds = (size_t)HB * Smax * 8;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_attention_gqa<VPF, NT, KP, DS, HB>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 8 * 256 * 8);
    attr_set = true;
  }
  hipLaunchKernelGGL((k_attention_gqa<VPF, NT, KP, DS, HB>), dim3(R, KV, DS), dim3(NT), lds, st, t, s, b, cos_t, sin_t, slot,
                     pos, kq, sk, v, exp_t, out, obits, H, KV, hd, Smax, INV, obn);
}
template <int HB>
static void att_gqa_go(int ds, int R, int H, size_t lds, hipStream_t st, const int64_t* t, const int32_t* s, const int64_t* b,
                       const int64_t* cos_t, const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq,
                       int32_t* sk, int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int KV, int hd, int Smax,
                       int INV, int obn) {
  if (ds == 4)
    att_gqa_go1<4, HB>(R, H, lds, st, t, s, b, cos_t, sin_t, slot, pos, kq, sk, v, exp_t, out, obits, KV, hd, Smax, INV, obn);
  else if (ds == 2)
    att_gqa_go1<2, HB>(R, H, lds, st, t, s, b, cos_t, sin_t, slot, pos, kq, sk, v, exp_t, out, obits, KV, hd, Smax, INV, obn);
  else
    att_gqa_go1<1, HB>(R, H, lds, st, t, s, b, cos_t, sin_t, slot, pos, kq, sk, v, exp_t, out, obits, KV, hd, Smax, INV, obn);
}

// blocks per (row, head) for the short-cache paths: the largest power of two up to ATT_DS that divides obn, keeps
// the launch in one round of ATT_WIDE_BLOCKS blocks and leaves a power of two of at most 64 value pairs a block
static int att_qkv_ds(int obn, int64_t blocks, int hd) {
  for (int ds = ATT_DS; ds > 1; ds >>= 1) {
    const int np = hd / (2 * ds);
    if (obn % ds == 0 && blocks * ds <= ATT_WIDE_BLOCKS && hd % (2 * ds) == 0 && np <= 64 && (np & (np - 1)) == 0)
      return ds;
  }
  return 1;
}

extern "C" int exact_attention_qkv_split(const int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                                         const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq,
                                         int32_t* sk, int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits,
                                         int32_t obn, int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t Smax, int32_t INV,
                                         void* stream) {
  if (!t || !s || !cos_t || !sin_t || !slot || !pos || !kq || !sk || !v || !exp_t || !out) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || hd <= 0 || Smax <= 0) return EXACT_E_ARG;
  if (obn != 1 && obn != 2 && obn != 4) return EXACT_E_ARG;
  if (hd > 256 || hd % 8 || (2 * ATT_THREADS) % hd || Smax > 8192) return EXACT_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(exp_t) & 15) return EXACT_E_ARG;   // staged into LDS in 16-byte pieces
  const size_t lds = (size_t)Smax * 8;
  const hipStream_t st = as_stream(stream);
  const int64_t blocks = (int64_t)R * H;
#define ATT_QKV_ARGS R, H, lds, st, t, s, b, cos_t, sin_t, slot, pos, kq, sk, v, exp_t, out, obits, KV, hd, Smax, INV, obn
  // caches of up to 2 ATT_WIDE_THREADS / 8 positions whose blocks fit one round: 8 threads per cached key (below), also
  // past ATT_VPF_LONG_S when ATT_KS8_LONG
  const bool ks8_wide = ATT_KS8 != 0 && ATT_KS8_WIDE_HD != 0 && hd % 64 == 0 && hd >= ATT_KS8_WIDE_HD && (2 * ATT_WIDE_THREADS) % hd == 0 &&
                        Smax <= 2 * (ATT_WIDE_THREADS / 8) && blocks <= ATT_WIDE_BLOCKS &&
                        (Smax <= ATT_VPF_LONG_S || ATT_KS8_LONG);
  // ... and of up to 4 ATT_WIDE_THREADS / 8 positions at hd 128 in four passes
  const bool ks8_wide4 = !ks8_wide && ATT_KS8 != 0 && ATT_KS8_LONG4 != 0 && hd == 128 && hd >= ATT_KS8_WIDE_HD &&
                         Smax <= 4 * (ATT_WIDE_THREADS / 8) && blocks <= ATT_WIDE_BLOCKS;
  const bool ks8_narrow = ATT_KS8 && hd % 64 == 0 && Smax <= 2 * (ATT_THREADS / 8);
  // blocks in several rounds (batched decode) over caches of up to 4 ATT_THREADS / 8 positions: ATT_THREADS-thread
  // blocks, 8 threads per cached key in two or four passes, exp table lookups from global memory (the LDS it would
  // take leaves room for more blocks per CU)
  const bool ks8_mr = ATT_KS8 && ATT_KS8_MR && blocks > ATT_WIDE_BLOCKS && hd % 64 == 0 && hd <= 128 &&
                      Smax <= 4 * (ATT_THREADS / 8);
  const int ds = ks8_wide || ks8_wide4 || (ks8_narrow && hd < ATT_KS8_WIDE_HD) ? att_qkv_ds(obn, blocks, hd) : 1;
  // ... and, for query groups of 4, 5, 7 or 8 heads over caches of at most 256 positions, one block per (row, KV
  // head, dimension slice) for the whole group
  const int grp = H / KV;
  const bool gqa = ATT_GQA && blocks > ATT_WIDE_BLOCKS && hd % 64 == 0 && hd <= 128 && Smax > ATT_GQA_MIN_S && Smax <= 256 &&
                   (grp == 4 || grp == 5 || grp == 7 || grp == 8);
  if (gqa) {
    const int gds = att_qkv_ds(obn, (int64_t)R * KV, hd);
    if (grp == 4) att_gqa_go<4>(gds, ATT_QKV_ARGS);
    else if (grp == 5) att_gqa_go<5>(gds, ATT_QKV_ARGS);
    else if (grp == 7) att_gqa_go<7>(gds, ATT_QKV_ARGS);
    else att_gqa_go<8>(gds, ATT_QKV_ARGS);
  } else if (ks8_mr) {
    if (Smax <= 2 * (ATT_THREADS / 8))
      att_qkv_go<ATT_MR_VPF, ATT_THREADS, ATT_KPF, 8, 2, 1, ATT_MR_GT != 0>(ATT_QKV_ARGS);
    else
      att_qkv_go<ATT_MR_VPF, ATT_THREADS, ATT_KPF, 8, 4, 1, ATT_MR_GT != 0>(ATT_QKV_ARGS);
  } else if (ks8_wide4) {
    // value prefetch: 2 ATT_WIDE_THREADS DS / hd threads per pair cover the up to 512 positions in VPF steps
    if (ds == 4)
      att_qkv_go<8, ATT_WIDE_THREADS, ATT_KPF, 8, 4, 4, ATT_GT1 != 0>(ATT_QKV_ARGS);
    else if (ds == 2)
      att_qkv_go<8, ATT_WIDE_THREADS, ATT_KPF, 8, 4, 2>(ATT_QKV_ARGS);
    else
      att_qkv_go<ATT_VPF, ATT_WIDE_THREADS, ATT_KPF, 8, 4>(ATT_QKV_ARGS);
  } else if (ATT_WIDE && !ks8_wide && Smax > ATT_VPF_LONG_S && blocks <= ATT_WIDE_BLOCKS && (2 * ATT_WIDE_THREADS) % hd == 0) {
    att_qkv_go<ATT_VPF_WIDE, ATT_WIDE_THREADS, 0>(ATT_QKV_ARGS);
  } else if (Smax > ATT_VPF_LONG_S && !ks8_wide) {
    att_qkv_go<ATT_VPF_LONG, ATT_THREADS>(ATT_QKV_ARGS);
  } else if (ks8_wide) {
    if (ds == 4)
      att_qkv_go<4, ATT_WIDE_THREADS, ATT_KPF, 8, 2, 4, ATT_GT1 != 0>(ATT_QKV_ARGS);
    else if (ds == 2)
      att_qkv_go<8, ATT_WIDE_THREADS, ATT_KPF, 8, 2, 2>(ATT_QKV_ARGS);
    else
      att_qkv_go<ATT_VPF, ATT_WIDE_THREADS, ATT_KPF, 8>(ATT_QKV_ARGS);
  } else if (ks8_narrow && hd < ATT_KS8_WIDE_HD) {
    if (ds == 4)
      att_qkv_go<2, ATT_THREADS, ATT_KPF, 8, 2, 4, ATT_GT1 != 0>(ATT_QKV_ARGS);
    else if (ds == 2)
      att_qkv_go<4, ATT_THREADS, ATT_KPF, 8, 2, 2>(ATT_QKV_ARGS);
    else
      att_qkv_go<ATT_VPF_NARROW, ATT_THREADS, ATT_KPF, 8>(ATT_QKV_ARGS);
  } else if (ks8_narrow) {
    att_qkv_go<ATT_VPF, ATT_THREADS, ATT_KPF, 8>(ATT_QKV_ARGS);
  } else {
    att_qkv_go<ATT_VPF, ATT_THREADS>(ATT_QKV_ARGS);
  }
#undef ATT_QKV_ARGS
  return launch_status("attention_qkv");
}

extern "C" int exact_attention_qkv(const int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                                   const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* kq, int32_t* sk,
                                   int64_t* v, const int32_t* exp_t, int64_t* out, int32_t* obits, int32_t R, int32_t H,
                                   int32_t KV, int32_t hd, int32_t Smax, int32_t INV, void* stream) {
  return exact_attention_qkv_split(t, s, b, cos_t, sin_t, slot, pos, kq, sk, v, exp_t, out, obits, 1, R, H, KV, hd, Smax,
                                   INV, stream);
}

extern "C" int exact_qkv_rope_cache(int64_t* t, const int32_t* s, const int64_t* b, const int64_t* cos_t,
                                    const int64_t* sin_t, const int32_t* slot, const int32_t* pos, int16_t* qq, int32_t* sq,
                                    int16_t* kq, int32_t* sk, int64_t* v, int32_t R, int32_t H, int32_t KV, int32_t hd,
                                    int32_t Smax, int32_t clear_t, void* stream) {
  if (!t || !s || !cos_t || !sin_t || !slot || !pos || !qq || !sq || !kq || !sk || !v) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || hd <= 0 || Smax <= 0) return EXACT_E_ARG;
  if (hd > 256 || hd % 2) return EXACT_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_qkv_rope_cache, dim3(R, H + 2 * KV), dim3(64), 0, as_stream(stream), t, s, b, cos_t, sin_t, slot,
                     pos, qq, sq, kq, sk, v, H, KV, hd, Smax, clear_t);
  return launch_status("qkv_rope_cache");
}

extern "C" int exact_attention(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                               const int64_t* v, const int32_t* slot, const int32_t* pos, const int32_t* exp_t,
                               int64_t* out, int32_t* obits, int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t Smax,
                               int32_t INV, void* stream) {
  if (!qq || !sq || !kq || !sk || !v || !slot || !pos || !exp_t || !out) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || hd <= 0 || Smax <= 0) return EXACT_E_ARG;
  if (hd > 256 || (2 * ATT_THREADS) % hd || hd % 8 || Smax > 8192) return EXACT_E_UNSUPPORTED;
  static bool attr_set = false;   // the scores take Smax * 8 bytes of LDS, up to 64 KiB beside the static arrays
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_attention<ATT_VPF, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 8192 * 8);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_attention<ATT_VPF_LONG, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 8192 * 8);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_attention<1, false>), hipFuncAttributeMaxDynamicSharedMemorySize,
                              8192 * 8);
    attr_set = true;
  }
  if (R * H > ATT_VPF_LONG_BLOCKS)
    hipLaunchKernelGGL((k_attention<1, false>), dim3(R, H), dim3(ATT_THREADS), (size_t)Smax * 8, as_stream(stream), qq, sq, kq, sk, v, slot,
                     pos,
                     exp_t, out, obits, H, KV, hd, Smax, INV);
  else if (Smax > ATT_VPF_LONG_S)
    hipLaunchKernelGGL((k_attention<ATT_VPF_LONG, true>), dim3(R, H), dim3(ATT_THREADS), (size_t)Smax * 8, as_stream(stream), qq, sq, kq, sk, v, slot,
                     pos,
                     exp_t, out, obits, H, KV, hd, Smax, INV);
  else
    hipLaunchKernelGGL((k_attention<ATT_VPF, true>), dim3(R, H), dim3(ATT_THREADS), (size_t)Smax * 8, as_stream(stream), qq, sq, kq, sk, v, slot,
                     pos,
                     exp_t, out, obits, H, KV, hd, Smax, INV);
  return launch_status("attention");
}
