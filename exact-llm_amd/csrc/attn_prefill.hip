// Exact integer attention for prefill on the matrix cores (gfx950): R query rows of one sequence, at
// increasing positions pos[r], against the keys 0..pos[r] of its cache slot. Same result as k_attention
// (exact_llm.py:170-176; exact_torch.py:142-166):
//   sc = shr((qq . kq) * INV, 32 - sq - sk); p = isoftmax(sc) (Q20); out = shr(p . v, 20)
//
// q.k from int8 digits on v_mfma_i32_32x32x32_i8. With x = 256 hi + lo + 128 (hi = x >> 8, lo = (x & 255) - 128,
// both int8):  q.k = 65536 HH + 256 (HL + LH) + LL + 128 (sum q + sum k) - 16384 hd; every digit product sum
// is below 2^22 in magnitude, so exact in int32.
// p.v from balanced int8 digits of p (p = d0 + 256 d1 + 65536 d2) and of v (4 digits when every |v| of the KV
// head is below 2^30, else 8): the digit products summed over the keys are exact in int32 when grouped by
// shift s = a + b, and p.v = sum_s C_s 256^s modulo 2^64, the reference's int64 product.
//
// The softmax needs the row maximum before any exponent and the row sum before any p, so k_attn_fused makes
// three passes over the keys of its 32 query rows, recomputing the scores on the matrix cores each time
// (cheaper than a round trip of int64 scores through HBM): max, then sum of exp, then p and p.v. The scores
// are computed transposed (keys x queries), so each lane holds one query row and 16 keys of a tile: the
// layout the p.v product takes p in, without a transpose. The V digits are stored with the keys of every
// 32-key group permuted to match (kdig/vdig below). Head dimension HD = 64 or 128 (a template parameter): the q.k
// products run over HD / 32 blocks of 32 dimensions and the p.v consumers take 32 dimensions each.
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace exact {


#define AP_TN 4608   // exp entries in LDS; the fast path needs the table to be zero from entry AP_TN - 2 on

// int16 -> (hi, lo - 128) int8 digits of 16 values held in two 16-byte chunks
__device__ __forceinline__ void split_digits(v4i p0, v4i p1, v4i& hi, v4i& lo) {
  hi[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x07050301u);
  hi[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x07050301u);
  hi[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x07050301u);
  hi[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x07050301u);
  lo[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x06040200u) ^ 0x80808080;
  lo[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x06040200u) ^ 0x80808080;
  lo[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x06040200u) ^ 0x80808080;
  lo[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x06040200u) ^ 0x80808080;
}

// sum of the 16 int16 values in two 16-byte chunks
__device__ __forceinline__ int sum16(v4i p0, v4i p1) {
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += (int)(int16_t)(p0[i] & 0xffff) + (int)(int16_t)(p0[i] >> 16);
    s += (int)(int16_t)(p1[i] & 0xffff) + (int)(int16_t)(p1[i] >> 16);
  }
  return s;
}

// V digits for the p.v product: vdig[(((kh * 8 + b) * ntile + t) * 2 + half) * hd + d][m] (16 bytes) is balanced
// base-256 digit b of v[32 t + 8 (m / 4) + 4 half + m % 4][d] (zero from nkeys on): the 16 keys in the order in
// which a transposed 32x32 MFMA result holds them for lane half `half`, and consecutive dimensions 16 bytes apart
// (so a wave's loads are contiguous). vpart[kh * ntile + t] = max bit length of |v| over the tile's keys.
// 2 HD threads work (the rest of the block only joins the reduction).
template <int HD>
__device__ __forceinline__ void vdigits_tile(const int64_t* __restrict__ v, int sl, int KV, int Smax, int nkeys, int kh, int t,
                                             int ntile, int8_t* __restrict__ vdig, int32_t* __restrict__ vpart, int* red) {
  const int d = threadIdx.x & (HD - 1), half = (threadIdx.x / HD) & 1;
  const bool act = threadIdx.x < 2 * HD;
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  v4i pk[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) pk[b] = v4i{};
  int bl = 0;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int key = 32 * t + 8 * (m >> 2) + 4 * half + (m & 3);
    int64_t x = act && key < nkeys ? v[(cbase + key) * HD + d] : 0;
    const int b0 = bitlen64(abs64(x));
    bl = b0 > bl ? b0 : bl;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int64_t dg = ((x + 128) & 255) - 128;
      pk[b][m >> 2] |= (int)(dg & 255) << (8 * (m & 3));
      x = (x - dg) >> 8;
    }
  }
  if (act)
#pragma unroll
    for (int b = 0; b < 8; ++b)
      *reinterpret_cast<v4i*>(vdig + (((((int64_t)kh * 8 + b) * ntile + t) * 2 + half) * HD + d) * 16) = pk[b];
  bl = block_max_i32(bl, red);
  if (threadIdx.x == 0) vpart[(int64_t)kh * ntile + t] = bl;
}

// Digits of every cached k of the sequence for the q.k product: kdig[(((kh * 2 + p) * HD / 32 + kb) * kpad + j) * 32 + c]
// = digit p (0: hi, 1: lo - 128) of k[j][32 kb + c]; ck[kh * kpad + j] = 128 sum_d k[j][d] - 16384 hd and
// skk[kh * kpad + j] = sk[j] (zeros from nkeys on); kpart[kh * ntile + t] = max sk over the tile's keys. The KV
// head 0 blocks also scan the exp table T, block t entries 256 t + [0, 256) (+ 8 kpad i): tpart[t] = 2^30 if one
// of them breaks the form the fast path takes (zero from entry AP_TN - 2 on, T[0] > 0, entries in [0, 2^24] with
// steps T[i] - T[i + 1] in [0, 2^24)), else 1 + the last nonzero index among them (0 if none). HD / 16 threads per
// key (16 dimensions each); the other threads of the block join the reductions and the table scan.
// Per-block results instead of global atomics: same-line atomics from every block serialise (~20 us here).
template <int HD>
__device__ __forceinline__ void kdigits_tile(const int16_t* __restrict__ kq, const int32_t* __restrict__ sk, int sl, int KV,
                                             int Smax, int nkeys, int kpad, int kh, int t, int8_t* __restrict__ kdig,
                                             int32_t* __restrict__ ck, int32_t* __restrict__ skk, int32_t* __restrict__ kpart,
                                             const int32_t* __restrict__ T, int32_t* __restrict__ tpart, int* red) {
  constexpr int TPK = HD / 16, KB = HD / 32;       // threads per key, 32-dimension blocks
  const int tid = threadIdx.x;
  const bool act = tid < 32 * TPK;
  const int j = 32 * t + tid / TPK, c = tid % TPK;   // c: 16 dimensions 16 c .. 16 c + 15
  const int64_t row = ((int64_t)sl * KV + kh) * Smax + j;
  v4i p0 = {}, p1 = {};
  if (act && j < nkeys) {
    const v4i* src = reinterpret_cast<const v4i*>(kq + row * HD + 16 * c);
    p0 = src[0];
    p1 = src[1];
  }
  v4i hi, lo;
  split_digits(p0, p1, hi, lo);
  if (j >= nkeys) lo = v4i{};
  const int kb = c >> 1, half = c & 1;
  if (act) {
    *reinterpret_cast<v4i*>(kdig + ((((int64_t)kh * 2 + 0) * KB + kb) * kpad + j) * 32 + 16 * half) = hi;
    *reinterpret_cast<v4i*>(kdig + ((((int64_t)kh * 2 + 1) * KB + kb) * kpad + j) * 32 + 16 * half) = lo;
  }
  int sum = sum16(p0, p1);
#pragma unroll
  for (int o = 1; o < TPK; o <<= 1) sum += __shfl_xor(sum, o, 64);
  int skv = 0;
  if (act && c == 0) {
    skv = j < nkeys ? sk[row] : 0;
    ck[(int64_t)kh * kpad + j] = j < nkeys ? 128 * sum - 16384 * HD : 0;
    skk[(int64_t)kh * kpad + j] = skv;
  }
  const int ntile = kpad / 32;
  skv = block_max_i32(skv, red);
  if (tid == 0) kpart[(int64_t)kh * ntile + t] = skv;
  if (kh == 0) {   // the fast path keeps exp entries [0, AP_TN) in LDS; the KV head 0 blocks scan the table
    int bad = 0, last = 0;
    for (int i = 256 * t + tid; i < EXACT_EXP_N; i += 8 * kpad) {
      const int x = T[i];
      if (i >= AP_TN - 2) {
        bad |= x != 0;
      } else {
        last = x != 0 ? i + 1 : last;
        const int y = T[i + 1];   // steps in [0, 2^24), entries in [0, 2^24], T[0] > 0
        bad |= y < 0 || x > (1 << 24) || x < y || x - y >= (1 << 24) || (i == 0 && x == 0);
      }
    }
    const int r = block_max_i32(bad ? 1 << 30 : last, red + 16);
    if (tid == 0) tpart[t] = r;
  }
}

// grid (kpad / 32, 2 KV), block 256: blocks with y < KV write V digits, the others k digits. part: the per-tile
// partial results, vpart [KV][kpad / 32], kpart [KV][kpad / 32], tpart [kpad / 32], every entry written here.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_digits(const int64_t* __restrict__ v, const int16_t* __restrict__ kq,
                                                     const int32_t* __restrict__ sk, const int32_t* __restrict__ T, int sl, int KV,
                                                     int Smax, int nkeys, int kpad, int8_t* __restrict__ vdig,
                                                     int8_t* __restrict__ kdig, int32_t* __restrict__ ck, int32_t* __restrict__ skk,
                                                     int32_t* __restrict__ part) {
  __shared__ int red[32];   // two reductions of 16 entries each
  const int ntile = kpad / 32;
  if ((int)blockIdx.y < KV)
    vdigits_tile<HD>(v, sl, KV, Smax, nkeys, blockIdx.y, blockIdx.x, ntile, vdig, part, red);
  else
    kdigits_tile<HD>(kq, sk, sl, KV, Smax, nkeys, kpad, blockIdx.y - KV, blockIdx.x, kdig, ck, skk, part + (int64_t)KV * ntile, T,
                 part + (int64_t)2 * KV * ntile, red);
}

// max of n int32 values, by every lane of a wave (the result is wave-uniform)
__device__ __forceinline__ int wave_max_of(const int32_t* __restrict__ a, int n) {
  int m = 0;   // every partial is >= 0
  for (int i = threadIdx.x & 63; i < n; i += 64) m = a[i] > m ? a[i] : m;
  return wave_max_i32(m);
}

// Raw buffer view of the n bytes at p (n < 2^31): a load's address is a per-lane 32-bit offset plus a wave-uniform
// scalar offset, so the tile loop spends no vector instructions on 64-bit addresses (loads past n read zeros).
typedef __amdgpu_buffer_rsrc_t BufRes;
__device__ __forceinline__ BufRes buf_res(const void* p, int64_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000);
}
__device__ __forceinline__ v4i buf_load16(BufRes r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// Scores of a tile (keys x queries) from the digit products: HH, HL + LH, LL.
struct QK {
  const int32_t* ckh;    // 128 sum k - 16384 hd per key
  const int32_t* skh;    // sk per key
  BufRes kdr;            // buffer view of this KV head's k digits
  BufRes kcr;            // one view from ckh to the end of skh (the key terms a wave loads one dword a lane)
  int kcoff;             // the lane's dword in it: ck of key l (l < 32), sk of key l - 32
  const v4i* qd;         // LDS q digits [kb][hi, lo][lane]: B operand, column = query l32, dimensions 32 kb + 16 half + [0, 16)
  // (kb < HD / 32; the callers pass HD as a template parameter)
  int kpad, l32, half, lane;
};

// k digits of one 32-key tile: A operand, row = key l32
template <int HD>
struct KTile {
  v4i hi[HD / 32], lo[HD / 32];
};

// per-key terms of the 16 keys a lane holds in a tile (keys j0 + 8 g + 4 half + [0, 4))
struct KCol {
  v4i ck[4], sk[4];
};

// The key terms of a tile at one dword a lane (lanes 0..31 ck of keys j0 + l, 32..63 sk of keys j0 + l - 32), put
// into the lane's own 16 keys through the wave's 256-byte LDS slot: 256 bytes of loads a tile instead of the 8 KiB
// that 16-byte loads of the lane's own keys take (the two half-waves hold different keys, so every lane of a half
// loads the same bytes).
__device__ __forceinline__ int load_kterm(const QK& c, int j0) {
  return __builtin_amdgcn_raw_buffer_load_b32(c.kcr, c.kcoff, j0 * 4, 0);
}
__device__ __forceinline__ void kterm_col(int32_t* slot, int kw, const QK& c, KCol& k) {
  slot[c.lane] = kw;
  __builtin_amdgcn_wave_barrier();   // the wave's own LDS write, read back by its other lanes (LDS is in order per wave)
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    k.ck[g] = *reinterpret_cast<const v4i*>(slot + 8 * g + 4 * c.half);
    k.sk[g] = *reinterpret_cast<const v4i*>(slot + 32 + 8 * g + 4 * c.half);
  }
}

template <int HD>
__device__ __forceinline__ void load_ktile(const QK& c, int j0, KTile<HD>& k) {
#pragma unroll
  for (int kb = 0; kb < HD / 32; ++kb) {
    k.hi[kb] = buf_load16(c.kdr, c.l32 * 32 + 16 * c.half, (kb * c.kpad + j0) * 32);
    k.lo[kb] = buf_load16(c.kdr, c.l32 * 32 + 16 * c.half, ((HD / 32 + kb) * c.kpad + j0) * 32);
  }
}

template <int HD>
__device__ __forceinline__ void mfma_ktile(const QK& c, const KTile<HD>& k, v16i& hh, v16i& xx, v16i& ll) {
  hh = v16i{};
  xx = v16i{};
  ll = v16i{};
#pragma unroll
  for (int kb = 0; kb < HD / 32; ++kb) {
    const v4i qh = c.qd[(2 * kb) * 64 + c.lane], ql = c.qd[(2 * kb + 1) * 64 + c.lane];
    hh = __builtin_amdgcn_mfma_i32_32x32x32_i8(k.hi[kb], qh, hh, 0, 0, 0);
    xx = __builtin_amdgcn_mfma_i32_32x32x32_i8(k.hi[kb], ql, xx, 0, 0, 0);
    xx = __builtin_amdgcn_mfma_i32_32x32x32_i8(k.lo[kb], qh, xx, 0, 0, 0);
    ll = __builtin_amdgcn_mfma_i32_32x32x32_i8(k.lo[kb], ql, ll, 0, 0, 0);
  }
}

// ---- float64 path. Exact when every |dot * INV| * 2^(sq + sk - 32) < 2^52, which the kernel checks over the
// block (sq + sk <= 33, INV < 2^14): dot < 2^38 and dot * INV < 2^52 are exact in float64, the power-of-two
// scalings are exact, and floor(w + 1/2) is shr's round-half-up. (256 HH + (HL + LH)) < 2^30 and
// LL + 128 (sum q + sum k) - 16384 hd < 2^31 are exact in int32.
#define AP_NEG (-1e300)

// max of two float64 values that are never NaN: one v_max_f64 (fmax adds NaN quieting)
__device__ __forceinline__ double max_f64(double a, double b) {
  double r;
  asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// unrounded score w (float64, exact) of an element; the score is floor(w + 1/2). SCALE false leaves out the row's
// factor fscale > 0 (the row maximum of w is the maximum of the unscaled values times fscale, and that product is
// exact for the same reason w is).
template <bool SCALE>
__device__ __forceinline__ double raw_score(int hh, int xx, int llc, double fscale, int skv) {
  const int m = (hh << 8) + xx;
  const double dot = __builtin_fma((double)m, 256.0, (double)llc);
  return __builtin_ldexp(SCALE ? dot * fscale : dot, skv);
}

// lut_exp(mx - sc) for mx - sc = dd >= 0 (exp16 below), given that T is zero from entry tz on (tz <= AP_TN - 2):
// indices past tz read entry tz (one address for every such lane, so the LDS read broadcasts), which also covers
// the reference's cut at 40.0. lim = 256 tz. dd = mx - floor(w + 1/2) = ceil((mx - 1/2) - w): w is N 2^-s with
// an integer |N| < 2^52 and s <= 32, so the difference is exact while below 2^53 2^-s, and a larger one (>= 2^21)
// clamps to lim either way.

// floor(e 2^20 / es) for 0 <= e <= es < 2^40 (es20 = es 2^-20, res20 = 2^20 / es rounded): the estimate
// e res20 - 2^-30 is below the quotient and within 2^-29 of it, so its floor is the result or one less; the
// remainder (e 2^20 - q es) 2^-20, exact in one fma (an integer below 2^41 over 2^20), is >= es20 in the second case.
// For e = 0 the estimate is -2^-30 and the correction brings -1 to 0.
__device__ __forceinline__ int pdiv_f64(int e, double es20, double res20) {
  const double ed = (double)e;
  const double q = __builtin_floor(__builtin_fma(ed, res20, -0x1p-30));
  const double r = __builtin_fma(-q, es20, ed);
  return (int)q + (r >= es20 ? 1 : 0);
}

// Balanced base-256 digits of p (0 <= p <= 2^20) for 4 keys at once: u = p + 128 + 128 * 256 holds d0 + 128,
// d1 + 128 and d2 in bytes 0, 1, 2; the planes take byte a of each u (planes 0 and 1 then flip bit 7).
__device__ __forceinline__ void pack_digits(int p0, int p1, int p2, int p3, int& w0, int& w1, int& w2) {
  const int u0 = p0 + 32896, u1 = p1 + 32896, u2 = p2 + 32896, u3 = p3 + 32896;
  const int y = __builtin_amdgcn_perm(u1, u0, 0x05010400u);   // u0.b0 u1.b0 u0.b1 u1.b1
  const int z = __builtin_amdgcn_perm(u3, u2, 0x05010400u);   // u2.b0 u3.b0 u2.b1 u3.b1
  const int y2 = __builtin_amdgcn_perm(u1, u0, 0x0c0c0602u);  // u0.b2 u1.b2 0 0
  const int z2 = __builtin_amdgcn_perm(u3, u2, 0x0c0c0602u);
  w0 = __builtin_amdgcn_perm(z, y, 0x05040100u) ^ 0x80808080;
  w1 = __builtin_amdgcn_perm(z, y, 0x07060302u) ^ 0x80808080;
  w2 = __builtin_amdgcn_perm(z2, y2, 0x05040100u);
}

struct FastCtx {
  const int32_t* T;   // LDS exp table
  double fscale;      // INV 2^(sq - 32)
  double tlim;        // 256 x the index from which the exp table is zero
  int rterm, mypos;
};

// the 16 unrounded scores of a tile (masked keys AP_NEG)
template <bool MASK, bool SCALE = true>
__device__ __forceinline__ void tile_raw(const QK& c, const FastCtx& f, int j0, const KCol& kc, const v16i& hh, const v16i& xx,
                                         const v16i& ll, double (&wv)[16]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const v4i ckv = kc.ck[g], skv = kc.sk[g];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 4 * g + u;
      double x = raw_score<SCALE>(hh[i], xx[i], ll[i] + ckv[u] + f.rterm, f.fscale, skv[u]);
      if (MASK) x = j0 + 8 * g + 4 * c.half + u <= f.mypos ? x : AP_NEG;
      wv[i] = x;
    }
  }
}

// running maximum of the unscaled scores (times fscale: the row's maximum w)
template <bool MASK>
__device__ __forceinline__ double tile_max(const QK& c, const FastCtx& f, int j0, const KCol& kc, const v16i& hh, const v16i& xx,
                                           const v16i& ll, double mw) {
  double wv[16];
  tile_raw<MASK, false>(c, f, j0, kc, hh, xx, ll, wv);
#pragma unroll
  for (int i = 0; i < 16; ++i) mw = max_f64(mw, wv[i]);
  return mw;
}

// exp_lds for the 16 elements of a tile with every LDS read issued before the first use; mxh = mx - 1/2. The table
// steps T[i] - T[i + 1] are in [0, 2^24) (checked with the table), so the interpolation product is a 24-bit one.
__device__ __forceinline__ void exp16(const int32_t* T, double mxh, const double (&wv)[16], double lim, int (&e)[16]) {
  int di[16], a[16], b[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) di[i] = (int)__builtin_fmin(__builtin_ceil(mxh - wv[i]), lim);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    a[i] = T[di[i] >> 8];
    b[i] = T[(di[i] >> 8) + 1];
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = a[i] - (int)((__umul24((unsigned)(a[i] - b[i]), (unsigned)(di[i] & 255)) + 128u) >> 8);
}

template <bool MASK>
__device__ __forceinline__ int tile_esum(const QK& c, const FastCtx& f, int j0, const KCol& kc, const v16i& hh, const v16i& xx,
                                         const v16i& ll, double mxh) {
  double wv[16];
  tile_raw<MASK>(c, f, j0, kc, hh, xx, ll, wv);
  int e[16];
  exp16(f.T, mxh, wv, f.tlim, e);
  int part = 0;   // 16 terms <= 2^24
#pragma unroll
  for (int i = 0; i < 16; ++i) part += e[i];
  return part;
}

template <bool MASK>
__device__ __forceinline__ void tile_pdig(const QK& c, const FastCtx& f, int j0, const KCol& kc, const v16i& hh, const v16i& xx,
                                          const v16i& ll, double mxh, double es20, double res20, v4i (&pa)[3]) {
  double wv[16];
  tile_raw<MASK>(c, f, j0, kc, hh, xx, ll, wv);
  int p[16];
  exp16(f.T, mxh, wv, f.tlim, p);
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = pdiv_f64(p[i], es20, res20);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
        int w0, w1, w2;
        pack_digits(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3], w0, w1, w2);
        pa[0][g] = w0;
        pa[1][g] = w1;
        pa[2][g] = w2;
      }
}

// ---- int64 path (any shifts, any exp table): shr64 and lut_exp as the reference, exp table in global memory
__device__ __forceinline__ void scores_i64(const QK& c, int j0, const v16i& hh, const v16i& xx, const v16i& ll, int64_t rterm,
                                           int sqv, int INV, int64_t (&sc)[16]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const v4i ckv = *reinterpret_cast<const v4i*>(c.ckh + j0 + 8 * g + 4 * c.half);
    const v4i skv = *reinterpret_cast<const v4i*>(c.skh + j0 + 8 * g + 4 * c.half);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 4 * g + u;
      const int64_t dot = ((int64_t)hh[i] << 16) + ((int64_t)xx[i] << 8) + (int64_t)(ll[i] + ckv[u]) + rterm;
      sc[i] = shr64(dot * INV, 32 - sqv - skv[u]);
    }
  }
}

#define AP_PROD 4      // the p.v kernel: waves 0..3 produce p digits, the HD / 32 waves after them multiply them into V
#define AP_SW 4        // waves of the statistics kernel

struct AttnLDS {
  int32_t* T;
  v4i (*Pl)[AP_PROD][3][64];
  int32_t* kcl;       // [waves][64]: each wave's key-term slot
  double* red_w;      // [waves][32]
  int64_t* red_a;     // [waves][32]
  int64_t* red_b;     // [waves][32]
};

// Consumer loop of the third pass: iteration s multiplies step s - 1 (the producers fill step s meanwhile). V digit
// plane b of tile t is at vr + voff + b vplane + 32 HD t. NB = 4 holds the V digits of a whole step and refills each
// tile's registers with the next step's tile once its products are issued; NB = 8 (no registers for that) loads one
// tile ahead.
template <int HD, int NB>
__device__ __forceinline__ void consume(const AttnLDS& L, int nsteps, int ntile, BufRes vr, int voff, int vplane, int lane,
                                        v16i (&acc)[NB + 2]) {
  auto load_v = [&](int t, v4i (&vb)[NB]) {
    t = t < ntile ? t : ntile - 1;   // stays inside the written keys
#pragma unroll
    for (int b = 0; b < NB; ++b) vb[b] = buf_load16(vr, voff, b * vplane + t * (2 * HD * 16));
  };
#pragma unroll
  for (int k = 0; k < NB + 2; ++k) acc[k] = v16i{};
  if constexpr (NB == 4) {
    v4i vb[AP_PROD][NB];
#pragma unroll
    for (int tt = 0; tt < AP_PROD; ++tt) load_v(tt, vb[tt]);
    for (int s = 0; s <= nsteps; ++s) {
      if (s >= 1) {
        const int buf = (s - 1) & 1, tiles = min(AP_PROD, ntile - AP_PROD * (s - 1));
#pragma unroll
        for (int tt = 0; tt < AP_PROD; ++tt) {
          if (tt < tiles) {
            v4i pv[3];
#pragma unroll
            for (int a = 0; a < 3; ++a) pv[a] = L.Pl[buf][tt][a][lane];
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
              for (int b = 0; b < NB; ++b) acc[a + b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pv[a], vb[tt][b], acc[a + b], 0, 0, 0);
          }
          if (s < nsteps) load_v(AP_PROD * s + tt, vb[tt]);
        }
      }
      __syncthreads();
    }
  } else {
    v4i vb[NB];
    load_v(0, vb);
    for (int s = 0; s <= nsteps; ++s) {
      if (s >= 1) {
        const int buf = (s - 1) & 1;
#pragma unroll 1
        for (int tt = 0; tt < AP_PROD && AP_PROD * (s - 1) + tt < ntile; ++tt) {
          const int t = AP_PROD * (s - 1) + tt;
          v4i pv[3], cur[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) cur[b] = vb[b];
          load_v(t + 1, vb);
#pragma unroll
          for (int a = 0; a < 3; ++a) pv[a] = L.Pl[buf][tt][a][lane];
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int a = 0; a < 3; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[a + b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pv[a], cur[b], acc[a + b], 0, 0, 0);
        }
      }
      __syncthreads();
    }
  }
}

// consume, then out = shr(sum_s C_s 256^s, 20) (modulo 2^64, as the reference's int64 p . v) for dimension d
// of the block's rows, and the rows' bit lengths in rowbits. C layout: lane holds rows 8 (i / 4) + 4 half + i % 4.
template <int HD, int NB>
__device__ __forceinline__ void consume_store(const AttnLDS& L, int nsteps, int ntile, BufRes vr, int voff, int vplane,
                                              int lane, int64_t* __restrict__ out, int* rowbits, int q0, int R, int H, int h, int d,
                                              int half) {
  v16i acc[NB + 2];
  consume<HD, NB>(L, nsteps, ntile, vr, voff, vplane, lane, acc);
  int b[16];   // bit length of |out| of row r(i) at this lane's dimension
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint64_t tot = 0;
#pragma unroll
    for (int k = 0; k < NB + 2; ++k) tot += (uint64_t)shl64((int64_t)acc[k][i], 8 * k);
    const int r = 8 * (i >> 2) + 4 * half + (i & 3);
    const int64_t o = shr64((int64_t)tot, 20);
    if (q0 + r < R) out[((int64_t)(q0 + r) * H + h) * HD + d] = o;
    b[i] = bitlen64(abs64(o));
  }
  // maxima over the 32 lanes (dimensions) of each half, transposed as they reduce: at the step over lane bit m the
  // lane keeps the upper or lower half of its values and takes its partner's other half, so after the bits 16, 8, 4,
  // 2 lane l holds row i = (l>>1&1) + 2 (l>>2&1) + 4 (l>>3&1) + 8 (l>>4&1) over 16 lanes, and bit 1 finishes it:
  // 16 shuffles and one LDS atomic per row and wave (a per-element atomic cost 7e6 bank conflicts per launch)
#pragma unroll
  for (int m = 16, n = 8; m >= 2; m >>= 1, n >>= 1) {
    const bool up = (lane & m) != 0;
#pragma unroll
    for (int j = 0; j < n; ++j) {
      const int other = __shfl_xor(up ? b[j] : b[j + n], m, 64);
      const int keep = up ? b[j + n] : b[j];
      b[j] = other > keep ? other : keep;
    }
  }
  const int other = __shfl_xor(b[0], 1, 64);
  if ((lane & 1) == 0) {
    const int i = ((lane >> 1) & 1) + 2 * ((lane >> 2) & 1) + 4 * ((lane >> 3) & 1) + 8 * ((lane >> 4) & 1);
    atomicMax(rowbits + 8 * (i >> 2) + 4 * half + (i & 3), other > b[0] ? other : b[0]);
  }
}

// Passes 1 and 2 for the float64 path: wave w of NW takes tiles w, w + NW, ...; the row maximum score and the
// row sum of exp. The per-key terms come in with each group of 4 keys (the statistics kernel runs 4 waves per
// SIMD, which hide the loads).
template <int HD, int NW>
__device__ __forceinline__ void passes12_f64(const QK& c, const AttnLDS& L, const FastCtx& f, int ntile, int firstpos, int w,
                                             double& mx, int64_t& es) {
  double mw = AP_NEG;
  int32_t* slot = L.kcl + 64 * w;
  KTile<HD> kt;   // the next tile's k digits and key terms load while this one is finished
  int kw = 0;
  if (w < ntile) {
    load_ktile(c, 32 * w, kt);
    kw = load_kterm(c, 32 * w);
  }
  for (int t = w; t < ntile; t += NW) {
    v16i hh, xx, ll;
    KCol kc;
    kterm_col(slot, kw, c, kc);   // LDS round trip under the products
    mfma_ktile(c, kt, hh, xx, ll);
    if (t + NW < ntile) {
      load_ktile(c, 32 * (t + NW), kt);
      kw = load_kterm(c, 32 * (t + NW));
    }
    __builtin_amdgcn_sched_barrier(0);
    mw = 32 * t + 31 <= firstpos ? tile_max<false>(c, f, 32 * t, kc, hh, xx, ll, mw) : tile_max<true>(c, f, 32 * t, kc, hh, xx, ll, mw);
  }
  mw = max_f64(mw, __shfl_xor(mw, 32, 64));
  if (c.half == 0) L.red_w[w * 32 + c.l32] = mw;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NW; ++k) mw = max_f64(mw, L.red_w[k * 32 + c.l32]);
  mx = __builtin_floor(mw * f.fscale + 0.5);
  const double mxh = mx - 0.5;
  int64_t e = 0;
  if (w < ntile) {
    load_ktile(c, 32 * w, kt);
    kw = load_kterm(c, 32 * w);
  }
  for (int t = w; t < ntile; t += NW) {
    v16i hh, xx, ll;
    KCol kc;
    kterm_col(slot, kw, c, kc);
    mfma_ktile(c, kt, hh, xx, ll);
    if (t + NW < ntile) {
      load_ktile(c, 32 * (t + NW), kt);
      kw = load_kterm(c, 32 * (t + NW));
    }
    __builtin_amdgcn_sched_barrier(0);
    e += 32 * t + 31 <= firstpos ? tile_esum<false>(c, f, 32 * t, kc, hh, xx, ll, mxh) : tile_esum<true>(c, f, 32 * t, kc, hh, xx, ll, mxh);
  }
  e += __shfl_xor(e, 32, 64);
  if (c.half == 0) L.red_a[w * 32 + c.l32] = e;
  __syncthreads();
  es = 0;
#pragma unroll
  for (int k = 0; k < NW; ++k) es += L.red_a[k * 32 + c.l32];
}

// Producer loop of the third pass (float64 path): iteration s turns tile AP_PROD s + w into p digits; the next
// tile's k digits and key terms load while this one is finished.
template <int HD>
__device__ __forceinline__ void produce_f64(const QK& c, const AttnLDS& L, const FastCtx& f, int nsteps, int ntile, int firstpos,
                                            int w, int lane, double mx, int64_t es) {
  const double es20 = __builtin_ldexp((double)es, -20), res20 = 1048576.0 / (double)es, mxh = mx - 0.5;
  KTile<HD> kt;
  int kw = 0;
  int32_t* slot = L.kcl + 64 * w;
  if (w < ntile) {
    load_ktile(c, 32 * w, kt);
    kw = load_kterm(c, 32 * w);
  }
  for (int s = 0; s <= nsteps; ++s) {
    const int t = AP_PROD * s + w;
    if (s < nsteps) {
      v4i pa[3] = {v4i{}, v4i{}, v4i{}};
      if (t < ntile) {
        v16i hh, xx, ll;
        KCol cur;
        kterm_col(slot, kw, c, cur);   // LDS round trip under the products
        mfma_ktile(c, kt, hh, xx, ll);
        if (t + AP_PROD < ntile) {
          load_ktile(c, 32 * (t + AP_PROD), kt);
          kw = load_kterm(c, 32 * (t + AP_PROD));
        }
        __builtin_amdgcn_sched_barrier(0);   // the next tile's loads in flight before this tile's epilogue
        if (32 * t + 31 <= firstpos) tile_pdig<false>(c, f, 32 * t, cur, hh, xx, ll, mxh, es20, res20, pa);
        else tile_pdig<true>(c, f, 32 * t, cur, hh, xx, ll, mxh, es20, res20, pa);
      }
#pragma unroll
      for (int a = 0; a < 3; ++a) L.Pl[s & 1][w][a][lane] = pa[a];
    }
    __syncthreads();
  }
}

// The int64 path (any shifts, any exp table): shr64 and lut_exp as the reference, exp table in global memory.
template <int HD, int NW>
__device__ __forceinline__ void passes12_i64(const QK& c, const AttnLDS& L, const int32_t* __restrict__ Tg, int64_t rterm, int sqv,
                                             int INV, int mypos, int ntile, int w, int64_t& mx, int64_t& es) {
  auto valid = [&](int t, int i) { return 32 * t + 8 * (i >> 2) + 4 * c.half + (i & 3) <= mypos; };
  int64_t m = INT64_MIN;
  for (int t = w; t < ntile; t += NW) {
    KTile<HD> kt;
    v16i hh, xx, ll;
    int64_t sc[16];
    load_ktile(c, 32 * t, kt);
    mfma_ktile(c, kt, hh, xx, ll);
    scores_i64(c, 32 * t, hh, xx, ll, rterm, sqv, INV, sc);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (valid(t, i)) m = sc[i] > m ? sc[i] : m;
  }
  {
    const int64_t o = __shfl_xor(m, 32, 64);
    m = o > m ? o : m;
  }
  if (c.half == 0) L.red_a[w * 32 + c.l32] = m;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NW; ++k) m = L.red_a[k * 32 + c.l32] > m ? L.red_a[k * 32 + c.l32] : m;
  mx = m;
  int64_t e = 0;
  for (int t = w; t < ntile; t += NW) {
    KTile<HD> kt;
    v16i hh, xx, ll;
    int64_t sc[16];
    load_ktile(c, 32 * t, kt);
    mfma_ktile(c, kt, hh, xx, ll);
    scores_i64(c, 32 * t, hh, xx, ll, rterm, sqv, INV, sc);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (valid(t, i)) e += lut_exp(Tg, mx - sc[i]);
  }
  e += __shfl_xor(e, 32, 64);
  if (c.half == 0) L.red_b[w * 32 + c.l32] = e;
  __syncthreads();
  es = 0;
#pragma unroll
  for (int k = 0; k < NW; ++k) es += L.red_b[k * 32 + c.l32];
}

template <int HD>
__device__ __forceinline__ void produce_i64(const QK& c, const AttnLDS& L, const int32_t* __restrict__ Tg, int64_t rterm, int sqv,
                                            int INV, int mypos, int nsteps, int ntile, int w, int lane, int64_t mx, int64_t es) {
  const double res = 1.0 / (double)es;
  for (int s = 0; s <= nsteps; ++s) {
    const int t = AP_PROD * s + w;
    if (s < nsteps) {
      v4i pa[3] = {v4i{}, v4i{}, v4i{}};
      if (t < ntile) {
        KTile<HD> kt;
        v16i hh, xx, ll;
        int64_t sc[16];
        load_ktile(c, 32 * t, kt);
        mfma_ktile(c, kt, hh, xx, ll);
        scores_i64(c, 32 * t, hh, xx, ll, rterm, sqv, INV, sc);
        int p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const bool ok = 32 * t + 8 * (i >> 2) + 4 * c.half + (i & 3) <= mypos;
          p[i] = ok ? (int)floordiv_rcp(shl64(lut_exp(Tg, mx - sc[i]), 20), es, res) : 0;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int w0, w1, w2;
          pack_digits(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3], w0, w1, w2);
          pa[0][g] = w0;
          pa[1][g] = w1;
          pa[2][g] = w2;
        }
      }
#pragma unroll
      for (int a = 0; a < 3; ++a) L.Pl[s & 1][w][a][lane] = pa[a];
    }
    __syncthreads();
  }
}

// What a block (32 query rows of one head) knows after set-up, in both kernels.
struct Block {
  QK c;
  int h, kh, q0, mypos, firstpos, ntile, sqs, sqv;
  int tz;      // 1 + the last nonzero index of the exp table (fast path)
  bool fast;
};

// Work item (query tile, head), heaviest tiles first. Workgroups go round-robin to the 8 XCDs (each with its own
// L2), so when KV divides 8, block b works on KV head (b % 8) % KV: each L2 then holds the k and v digits of one
// KV head. Item j of a KV head is query tile nqt - 1 - j / hq of head kh hq + j % hq. Returns false for the
// blocks past the work (the grid is rounded up to a multiple of 8).
__device__ __forceinline__ bool block_item(int R, int H, int KV, int& h, int& kh, int& q0) {
  const int nqt = (R + 31) / 32, hq = H / KV;
  int j;
  if (8 % KV == 0) {
    kh = (blockIdx.x & 7) % KV;
    j = (blockIdx.x >> 3) * (8 / KV) + (blockIdx.x & 7) / KV;
  } else {
    kh = (blockIdx.x % H) / hq;
    j = (blockIdx.x / H) * hq + (blockIdx.x % H) % hq;
  }
  if (j >= nqt * hq) return false;
  h = kh * hq + j % hq;
  q0 = (nqt - 1 - j / hq) * 32;
  return true;
}

// Loads the exp table and the q digits into LDS (ends with a barrier) and fills b. part: k_attn_digits' per-tile
// results. The float64 decision depends only on the block's rows, so both kernels agree.
template <int HD>
__device__ __forceinline__ void block_setup(Block& b, int h, int kh, int q0, const int16_t* __restrict__ qq,
                                            const int32_t* __restrict__ sq, const int8_t* __restrict__ kdig,
                                            const int32_t* __restrict__ ck, const int32_t* __restrict__ skk,
                                            const int32_t* __restrict__ part, const int32_t* __restrict__ pos,
                                            const int32_t* __restrict__ Tg, int32_t* T, v4i (*Qd)[64], int R, int H, int KV,
                                            int nkeys, int kpad, int INV) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  {   // exp table into LDS, 16 bytes a lane, every load issued before the first store (blocks of 256 or 512)
    constexpr int NV = AP_TN / 4, NK = (NV + 255) / 256;
    v4i r[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int i = tid + k * (int)blockDim.x;
      if (i < NV) r[k] = reinterpret_cast<const v4i*>(Tg)[i];
    }
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int i = tid + k * (int)blockDim.x;
      if (i < NV) reinterpret_cast<v4i*>(T)[i] = r[k];
    }
  }
  b.h = h;
  b.kh = kh;
  b.q0 = q0;
  QK& c = b.c;
  c.l32 = lane & 31;
  c.half = lane >> 5;
  c.lane = lane;
  c.qd = &Qd[0][0];
  c.kpad = kpad;
  c.ckh = ck + (int64_t)kh * kpad;
  c.skh = skk + (int64_t)kh * kpad;
  c.kdr = buf_res(kdig + (int64_t)kh * 2 * HD * kpad, (int64_t)2 * HD * kpad);   // 2 digits x HD / 32 blocks x kpad x 32
  {
    const int64_t d = reinterpret_cast<const char*>(c.skh) - reinterpret_cast<const char*>(c.ckh);   // > 0, < 2^31
    c.kcr = buf_res(c.ckh, d + (int64_t)kpad * 4);
    c.kcoff = lane < 32 ? 4 * lane : (int)d + 4 * (lane - 32);
  }
  const int qr = q0 + c.l32 < R ? q0 + c.l32 : R - 1;
  const int qlast = q0 + 31 < R ? q0 + 31 : R - 1;
  const int jmax = max(0, min(pos[qlast], nkeys - 1));       // positions increase with the row
  b.firstpos = max(0, min(pos[q0], nkeys - 1));
  b.mypos = max(0, min(pos[qr], nkeys - 1));
  b.ntile = jmax / 32 + 1;
  int sqs = 0;
  const v4i* qp = reinterpret_cast<const v4i*>(qq + ((int64_t)qr * H + h) * HD);
#pragma unroll
  for (int kb = 0; kb < HD / 32; ++kb) {
    const v4i a0 = qp[(32 * kb + 16 * c.half) / 8], a1 = qp[(32 * kb + 16 * c.half) / 8 + 1];
    v4i qh, ql;
    split_digits(a0, a1, qh, ql);
    if (w == 0) {   // every wave holds the same rows
      Qd[2 * kb][lane] = qh;
      Qd[2 * kb + 1][lane] = ql;
    }
    sqs += sum16(a0, a1);
  }
  b.sqs = sqs + __shfl_xor(sqs, 32, 64);
  b.sqv = sq[(int64_t)qr * H + h];
  // uniform over the block: every wave sees the same 32 rows and reduces the same partials
  const int nt = kpad / 32;
  const int skmax = wave_max_of(part + (int64_t)(KV + kh) * nt, nt), tab = wave_max_of(part + (int64_t)2 * KV * nt, nt);
  b.tz = tab;
  b.fast = wave_max_i32(b.sqv) + skmax <= 33 && INV >= 0 && INV < (1 << 14) && tab < (1 << 30);
  __syncthreads();
}

// Passes 1 and 2 (row maximum score, row sum of exp). grid as k_attn_pv, block 64 AP_SW. st_mx / st_es: [H][R]
// int64 (the float64 path stores its exact integer maximum as an int64 too).
template <int HD>
__global__ __launch_bounds__(64 * AP_SW, 3) void k_attn_stats(const int16_t* __restrict__ qq, const int32_t* __restrict__ sq,
                                                              const int8_t* __restrict__ kdig, const int32_t* __restrict__ ck,
                                                              const int32_t* __restrict__ skk, const int32_t* __restrict__ part,
                                                              const int32_t* __restrict__ pos, const int32_t* __restrict__ Tg,
                                                              int64_t* __restrict__ st_mx, int64_t* __restrict__ st_es, int R,
                                                              int H, int KV, int nkeys, int kpad, int INV) {
  __shared__ __attribute__((aligned(16))) int32_t T[AP_TN];
  __shared__ v4i Qd[HD / 16][64];
  __shared__ double red_w[AP_SW * 32];
  __shared__ int64_t red_a[AP_SW * 32], red_b[AP_SW * 32];
  __shared__ __attribute__((aligned(16))) int32_t kcl[AP_SW * 64];
  int h, kh, q0;
  if (!block_item(R, H, KV, h, kh, q0)) return;
  Block b;
  block_setup<HD>(b, h, kh, q0, qq, sq, kdig, ck, skk, part, pos, Tg, T, Qd, R, H, KV, nkeys, kpad, INV);
  const int w = threadIdx.x >> 6;
  AttnLDS L{T, nullptr, kcl, red_w, red_a, red_b};
  int64_t mx, es;
  if (b.fast) {
    const FastCtx f{T, __builtin_ldexp((double)INV, b.sqv - 32), 256.0 * b.tz, 128 * b.sqs, b.mypos};
    double m;
    passes12_f64<HD, AP_SW>(b.c, L, f, b.ntile, b.firstpos, w, m, es);
    mx = (int64_t)m;
  } else {
    passes12_i64<HD, AP_SW>(b.c, L, Tg, 128 * (int64_t)b.sqs, b.sqv, INV, b.mypos, b.ntile, w, mx, es);
  }
  const int row = q0 + b.c.l32;
  if (w == 0 && b.c.half == 0 && row < R) {
    st_mx[(int64_t)h * R + row] = mx;
    st_es[(int64_t)h * R + row] = es;
  }
}

// Pass 3. grid ceil(R / 32) H rounded up to a multiple of 8, block 512 (8 waves): 32 query rows of one head per
// block, heaviest tiles first. In steps of 4 key tiles of 32, waves 0..3 turn tile 4 s + w into p digits (LDS,
// double-buffered) while the HD / 32 waves after them multiply the previous step's p into V, each for 32 dimensions
// (at HD 128 a producer and a consumer share each SIMD). The consumers use 4 V digits when every |v| of the KV head
// is below 2^30, else 8.
template <int HD>
__global__ __launch_bounds__(64 * (AP_PROD + HD / 32)) void k_attn_pv(const int16_t* __restrict__ qq, const int32_t* __restrict__ sq,
                                                 const int8_t* __restrict__ kdig, const int32_t* __restrict__ ck,
                                                 const int32_t* __restrict__ skk, const int32_t* __restrict__ part,
                                                 const int8_t* __restrict__ vdig, const int32_t* __restrict__ pos,
                                                 const int32_t* __restrict__ Tg, const int64_t* __restrict__ st_mx,
                                                 const int64_t* __restrict__ st_es, int64_t* __restrict__ out,
                                                 int32_t* __restrict__ obits, int R, int H, int KV, int nkeys, int kpad,
                                                 int INV) {
  __shared__ __attribute__((aligned(16))) int32_t T[AP_TN];
  __shared__ v4i Pl[2][AP_PROD][3][64];
  __shared__ v4i Qd[HD / 16][64];
  __shared__ int rowbits[32];
  __shared__ __attribute__((aligned(16))) int32_t kcl[AP_PROD * 64];
  int h, kh, q0;
  if (!block_item(R, H, KV, h, kh, q0)) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  if (tid < 32) rowbits[tid] = 0;
  Block b;
  block_setup<HD>(b, h, kh, q0, qq, sq, kdig, ck, skk, part, pos, Tg, T, Qd, R, H, KV, nkeys, kpad, INV);
  const QK& c = b.c;
  const int row = q0 + c.l32 < R ? q0 + c.l32 : R - 1;
  const int64_t mx = st_mx[(int64_t)h * R + row], es = st_es[(int64_t)h * R + row];
  AttnLDS L{T, Pl, kcl, nullptr, nullptr, nullptr};
  const int nsteps = (b.ntile + AP_PROD - 1) / AP_PROD;
  const int dc = w - AP_PROD;   // consumer: dimensions 32 dc + [0, 32)
  const int vplane = HD * kpad;   // one digit plane: kpad / 32 tiles x 2 halves x hd x 16 bytes
  const BufRes vr = buf_res(vdig + (int64_t)kh * 8 * vplane, (int64_t)8 * vplane);
  const int voff = (c.half * HD + 32 * dc + c.l32) * 16;
  if (w >= AP_PROD) {
    if (wave_max_of(part + (int64_t)kh * (kpad / 32), kpad / 32) + 2 <= 32)
      consume_store<HD, 4>(L, nsteps, b.ntile, vr, voff, vplane, lane, out, rowbits, q0, R, H, h, 32 * dc + c.l32, c.half);
    else
      consume_store<HD, 8>(L, nsteps, b.ntile, vr, voff, vplane, lane, out, rowbits, q0, R, H, h, 32 * dc + c.l32, c.half);
  } else if (b.fast) {
    const FastCtx f{T, __builtin_ldexp((double)INV, b.sqv - 32), 256.0 * b.tz, 128 * b.sqs, b.mypos};
    produce_f64<HD>(c, L, f, nsteps, b.ntile, b.firstpos, w, lane, (double)mx, es);
  } else {
    produce_i64<HD>(c, L, Tg, 128 * (int64_t)b.sqs, b.sqv, INV, b.mypos, nsteps, b.ntile, w, lane, mx, es);
  }
  __syncthreads();
  if (obits && tid < 32 && q0 + tid < R) obits[(int64_t)(q0 + tid) * H + h] = rowbits[tid];
}

// workspace layout (bytes, each part 256-aligned): vdig KV*8*hd*kpad, kdig KV*2*hd*kpad, ck and skk KV*kpad*4
// each, the digit kernel's per-tile results (2 KV + 1) * kpad / 32 int32; row maxima and sums H*R*8 each
static int64_t al256(int64_t n) { return (n + 255) & ~(int64_t)255; }
static int64_t ws_bytes(int R, int H, int KV, int hd, int kpad) {
  return al256((int64_t)KV * 8 * hd * kpad) + al256((int64_t)KV * 2 * hd * kpad) + 2 * al256((int64_t)KV * kpad * 4) +
         al256((int64_t)(2 * KV + 1) * (kpad / 32) * 4) + 2 * al256((int64_t)H * R * 8);
}

}  // namespace exact

using namespace exact;

extern "C" int64_t exact_attention_prefill_workspace(int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t nkeys) {
  if (R <= 0 || H <= 0 || KV <= 0 || (hd != 64 && hd != 128) || nkeys <= 0) return -1;
  return ws_bytes(R, H, KV, hd, (nkeys + 31) / 32 * 32);
}

extern "C" int exact_attention_prefill(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                                       const int64_t* v, int32_t slot, const int32_t* pos, const int32_t* exp_t, int64_t* out,
                                       int32_t* obits, void* work, int64_t work_bytes, int32_t R, int32_t H, int32_t KV,
                                       int32_t hd, int32_t Smax, int32_t nkeys, int32_t INV, void* stream) {
  if (!qq || !sq || !kq || !sk || !v || !pos || !exp_t || !out || !work) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || slot < 0 || Smax <= 0 || nkeys <= 0 || nkeys > Smax) return EXACT_E_ARG;
  // per shift class, 3 digit pairs x nkeys products of |.| <= 2^14 stay below 2^31
  if ((hd != 64 && hd != 128) || nkeys > 32768) return EXACT_E_UNSUPPORTED;
  const int kpad = (nkeys + 31) / 32 * 32;
  if (work_bytes < ws_bytes(R, H, KV, hd, kpad) || (reinterpret_cast<uintptr_t>(work) & 255) ||
      (reinterpret_cast<uintptr_t>(exp_t) & 15))
    return EXACT_E_ARG;
  int8_t* vdig = static_cast<int8_t*>(work);
  int8_t* kdig = vdig + al256((int64_t)KV * 8 * hd * kpad);
  int32_t* ck = reinterpret_cast<int32_t*>(kdig + al256((int64_t)KV * 2 * hd * kpad));
  int32_t* skk = reinterpret_cast<int32_t*>(reinterpret_cast<int8_t*>(ck) + al256((int64_t)KV * kpad * 4));
  int32_t* part = reinterpret_cast<int32_t*>(reinterpret_cast<int8_t*>(skk) + al256((int64_t)KV * kpad * 4));
  int64_t* st_mx = reinterpret_cast<int64_t*>(reinterpret_cast<int8_t*>(part) + al256((int64_t)(2 * KV + 1) * (kpad / 32) * 4));
  int64_t* st_es = reinterpret_cast<int64_t*>(reinterpret_cast<int8_t*>(st_mx) + al256((int64_t)H * R * 8));
  hipStream_t st = as_stream(stream);
  const dim3 grid(((R + 31) / 32 * H + 7) / 8 * 8);
#define AP_GO(HD)                                                                                                      \
  do {                                                                                                                 \
    hipLaunchKernelGGL(k_attn_digits<HD>, dim3(kpad / 32, 2 * KV), dim3(256), 0, st, v, kq, sk, exp_t, slot, KV, Smax,   \
                       nkeys, kpad, vdig, kdig, ck, skk, part);                                                        \
    hipLaunchKernelGGL(k_attn_stats<HD>, grid, dim3(64 * AP_SW), 0, st, qq, sq, kdig, ck, skk, part, pos, exp_t, st_mx,  \
                       st_es, R, H, KV, nkeys, kpad, INV);                                                             \
    hipLaunchKernelGGL(k_attn_pv<HD>, grid, dim3(64 * (AP_PROD + HD / 32)), 0, st, qq, sq, kdig, ck, skk, part, vdig,    \
                       pos, exp_t, st_mx, st_es, out, obits, R, H, KV, nkeys, kpad, INV);                              \
  } while (0)
  if (hd == 64)
    AP_GO(64);
  else
    AP_GO(128);
#undef AP_GO
  return launch_status("attention_prefill");
}
