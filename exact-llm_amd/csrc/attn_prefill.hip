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
// 32-key group permuted to match (kdig/vdig below). Head dimension 128.
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace exact {

int zero_bytes(void* dst, int64_t nbytes, hipStream_t st);

#define AP_HD 128

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

// Position of key jj (0..31) inside its 32-key group in kdig/vdig order: the group is stored as the keys
// 8c + 4h + u (u < 4) at 16 h + 4 c + u, so half h of a wave reads its 16 keys as one 16-byte chunk, in the order
// 8 (m / 4) + 4 h + m % 4 (m = byte) in which a transposed 32x32 MFMA result holds them.
__device__ __forceinline__ int key_slot(int jj) { return 16 * ((jj >> 2) & 1) + 4 * (jj >> 3) + (jj & 3); }

// Balanced base-256 digits of every v of the sequence, transposed: vdig[((kh * 8 + b) * hd + d) * kpad + slot]
// (slot: key_slot inside each 32-key group; zeros from nkeys on); vbits[kh] = max bit length of |v| over the
// KV head (zeroed before). grid (kpad / 32, KV), block 256: 32 keys read row-major, staged in LDS, written 32
// keys per (digit, dimension).
#define VD_STRIDE 36   // bytes per LDS row of 32 keys, padded against bank conflicts
__global__ __launch_bounds__(256) void k_vdigits(const int64_t* __restrict__ v, int sl, int KV, int Smax, int nkeys, int kpad,
                                                 int8_t* __restrict__ vdig, int32_t* __restrict__ vbits) {
  __shared__ __align__(16) int8_t st[8 * AP_HD * VD_STRIDE];
  const int kh = blockIdx.y, j0 = blockIdx.x * 32, tid = threadIdx.x;
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  int bl = 0;
#pragma unroll 4
  for (int i = 0; i < 32 * AP_HD / 256; ++i) {
    const int e = tid + 256 * i, key = e / AP_HD, d = e % AP_HD;
    int64_t x = j0 + key < nkeys ? v[(cbase + j0 + key) * AP_HD + d] : 0;
    const int b0 = bitlen64(abs64(x));
    bl = b0 > bl ? b0 : bl;
    const int slot = key_slot(key);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int64_t dg = ((x + 128) & 255) - 128;
      st[(b * AP_HD + d) * VD_STRIDE + slot] = (int8_t)dg;
      x = (x - dg) >> 8;
    }
  }
  bl = wave_max_i32(bl);
  if ((tid & 63) == 0) atomicMax(vbits + kh, bl);
  __syncthreads();
  int8_t* dst = vdig + (int64_t)kh * 8 * AP_HD * kpad + j0;
#pragma unroll 4
  for (int i = 0; i < 8 * AP_HD * 8 / 256; ++i) {
    const int idx = tid + 256 * i, row = idx >> 3, w = idx & 7;   // row = b * hd + d, w = dword of 32 keys
    *reinterpret_cast<int32_t*>(dst + (int64_t)row * kpad + 4 * w) = *reinterpret_cast<const int32_t*>(st + row * VD_STRIDE + 4 * w);
  }
}

// Digits of every cached k of the sequence for the q.k product: kdig[(((kh * 2 + p) * 4 + kb) * kpad + j) * 32 + c]
// = digit p (0: hi, 1: lo - 128) of k[j][32 kb + c]; ck[kh * kpad + j] = 128 sum_d k[j][d] - 16384 hd and
// skk[kh * kpad + j] = sk[j] (zeros from nkeys on); skmax[kh] = max sk (zeroed before). grid (kpad / 32, KV),
// block 256: 8 threads per key.
__global__ __launch_bounds__(256) void k_kdigits(const int16_t* __restrict__ kq, const int32_t* __restrict__ sk, int sl, int KV,
                                                 int Smax, int nkeys, int kpad, int8_t* __restrict__ kdig, int32_t* __restrict__ ck,
                                                 int32_t* __restrict__ skk, int32_t* __restrict__ skmax) {
  const int kh = blockIdx.y, tid = threadIdx.x;
  const int j = blockIdx.x * 32 + (tid >> 3), c = tid & 7;   // c: 16 dimensions 16 c .. 16 c + 15
  const int64_t row = ((int64_t)sl * KV + kh) * Smax + j;
  v4i p0 = {}, p1 = {};
  if (j < nkeys) {
    const v4i* src = reinterpret_cast<const v4i*>(kq + row * AP_HD + 16 * c);
    p0 = src[0];
    p1 = src[1];
  }
  v4i hi, lo;
  split_digits(p0, p1, hi, lo);
  if (j >= nkeys) lo = v4i{};
  const int kb = c >> 1, half = c & 1;
  *reinterpret_cast<v4i*>(kdig + ((((int64_t)kh * 2 + 0) * 4 + kb) * kpad + j) * 32 + 16 * half) = hi;
  *reinterpret_cast<v4i*>(kdig + ((((int64_t)kh * 2 + 1) * 4 + kb) * kpad + j) * 32 + 16 * half) = lo;
  int sum = sum16(p0, p1);
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  sum += __shfl_xor(sum, 4, 64);
  int skv = 0;
  if (c == 0) {
    skv = j < nkeys ? sk[row] : 0;
    ck[(int64_t)kh * kpad + j] = j < nkeys ? 128 * sum - 16384 * AP_HD : 0;
    skk[(int64_t)kh * kpad + j] = skv;
  }
  skv = wave_max_i32(skv);
  if ((tid & 63) == 0) atomicMax(skmax + kh, skv);
}

// floor(a / b) for b > 0 given rb ~ 1 / b: the estimate is corrected exactly, as in floordiv_pos
__device__ __forceinline__ int64_t floordiv_rcp(int64_t a, int64_t b, double rb) {
  double qd = __builtin_floor((double)a * rb);
  qd = qd > 9.2e18 ? 9.2e18 : (qd < -9.2e18 ? -9.2e18 : qd);
  int64_t q = (int64_t)qd;
  int64_t r = (int64_t)((uint64_t)a - (uint64_t)q * (uint64_t)b);
  while (r < 0) { --q; r += b; }
  while (r >= b) { ++q; r -= b; }
  return q;
}

// Scores of a tile (keys x queries) from the digit products: HH, HL + LH, LL.
struct QK {
  const int8_t* kd;      // this KV head's k digits
  const int32_t* ckh;    // 128 sum k - 16384 hd per key
  const int32_t* skh;    // sk per key
  int kpad, l32, half;
  v4i qh[4], ql[4];      // q digits: B operand, column = query l32, dimensions 32 kb + 16 half + [0, 16)
};

__device__ __forceinline__ void qk_tile(const QK& c, int j0, v16i& hh, v16i& xx, v16i& ll) {
  hh = v16i{};
  xx = v16i{};
  ll = v16i{};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const v4i khi = *reinterpret_cast<const v4i*>(c.kd + ((int64_t)kb * c.kpad + j0 + c.l32) * 32 + 16 * c.half);
    const v4i klo = *reinterpret_cast<const v4i*>(c.kd + ((int64_t)(4 + kb) * c.kpad + j0 + c.l32) * 32 + 16 * c.half);
    hh = __builtin_amdgcn_mfma_i32_32x32x32_i8(khi, c.qh[kb], hh, 0, 0, 0);
    xx = __builtin_amdgcn_mfma_i32_32x32x32_i8(khi, c.ql[kb], xx, 0, 0, 0);
    xx = __builtin_amdgcn_mfma_i32_32x32x32_i8(klo, c.qh[kb], xx, 0, 0, 0);
    ll = __builtin_amdgcn_mfma_i32_32x32x32_i8(klo, c.ql[kb], ll, 0, 0, 0);
  }
}

// Float64 scores, exact when every |dot * INV| * 2^(sq + sk - 32) < 2^52 (the kernel checks sq + sk <= 33 and
// INV < 2^14 over the block): dot < 2^38 and dot * INV < 2^52 are exact, the power-of-two scalings are exact,
// and floor(w + 1/2) is shr's round-half-up. Masked keys (past the row's position) get -1e300.
#define AP_NEG (-1e300)
template <bool MASK>
__device__ __forceinline__ void scores_f64(const QK& c, int j0, int rterm, double fscale, int mypos, double (&sc)[16]) {
  v16i hh, xx, ll;
  qk_tile(c, j0, hh, xx, ll);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const v4i ckv = *reinterpret_cast<const v4i*>(c.ckh + j0 + 8 * g + 4 * c.half);
    const v4i skv = *reinterpret_cast<const v4i*>(c.skh + j0 + 8 * g + 4 * c.half);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = 4 * g + u;
      const double d = __builtin_fma((double)hh[i], 65536.0, __builtin_fma((double)xx[i], 256.0, (double)(ll[i] + ckv[u] + rterm)));
      double w = __builtin_floor(__builtin_ldexp(d * fscale, skv[u]) + 0.5);
      if (MASK) w = j0 + 8 * g + 4 * c.half + u <= mypos ? w : AP_NEG;
      sc[i] = w;
    }
  }
}

// exp LUT of mx - sc (>= 0, exact in float64): lut_exp without 64-bit integer work; 0 for masked keys
__device__ __forceinline__ int exp_f64(const int32_t* T, double mx, double sc) {
  const double dd = mx - sc;
  const int di = (int)__builtin_fmin(dd, (double)((40 << EXACT_F) - 1));
  const int i = di >> 8, fr = di & 255;
  const int a = T[i], b = T[i + 1];
  const int e = a - (((a - b) * fr + 128) >> 8);
  return dd < (double)(40 << EXACT_F) ? e : 0;
}

// floor(e 2^20 / es) for 0 <= e <= 2^24 < es... : the estimate e 2^20 * (1 / es) is within 2^-31 of the quotient,
// and the remainder (exact in float64, below 2^53) corrects it by one either way.
__device__ __forceinline__ int pdiv_f64(int e, double es, double res) {
  const double a = (double)e * 1048576.0;
  double q = __builtin_floor(a * res);
  const double r = __builtin_fma(-q, es, a);
  q = r < 0.0 ? q - 1.0 : q;
  q = r >= es ? q + 1.0 : q;
  return (int)q;
}

// int64 scores (any sq, sk): shr64 as the reference
__device__ __forceinline__ void scores_i64(const QK& c, int j0, int64_t rterm, int sqv, int INV, int64_t (&sc)[16]) {
  v16i hh, xx, ll;
  qk_tile(c, j0, hh, xx, ll);
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

// byte i % 4 of word i / 4 of the three balanced digit planes of p (0 <= p <= 2^20); planes 0 and 1 still
// carry +128 (flipped by the caller with ^ 0x80808080)
__device__ __forceinline__ void put_digits(int p, int i, v4i (&pa)[3]) {
  const int t0 = p + 128;
  const int t1 = (t0 >> 8) + 128;
  const int sh = 8 * (i & 3);
  pa[0][i >> 2] |= (t0 & 255) << sh;
  pa[1][i >> 2] |= (t1 & 255) << sh;
  pa[2][i >> 2] |= (t1 >> 8) << sh;
}

struct AttnLDS {
  int32_t* T;
  v4i (*Pl)[4][3][64];
  int64_t (*red_mx)[32];
  int64_t (*red_es)[32];
  int* rowbits;
};

template <int NB, bool FAST>
__device__ __forceinline__ void attn_body(const QK& c, const AttnLDS& L, int64_t rterm, int sqv, int INV, int mypos,
                                          int ntile, int firstpos, const int8_t* __restrict__ vd, int64_t vplane,
                                          int w, int lane, v16i (&acc)[NB + 2]) {
  const int l32 = c.l32, half = c.half;
  const int rt32 = (int)rterm;
  const double fscale = __builtin_ldexp((double)INV, sqv - 32);
  // pass 1: row maximum
  int64_t mx;
  double mxd = AP_NEG;
  if (FAST) {
    for (int t = w; t < ntile; t += 4) {
      double sc[16];
      if (32 * t + 31 <= firstpos) scores_f64<false>(c, 32 * t, rt32, fscale, mypos, sc);
      else scores_f64<true>(c, 32 * t, rt32, fscale, mypos, sc);
#pragma unroll
      for (int i = 0; i < 16; ++i) mxd = __builtin_fmax(mxd, sc[i]);
    }
    mxd = __builtin_fmax(mxd, __shfl_xor(mxd, 32, 64));
    mx = (int64_t)mxd;
  } else {
    mx = INT64_MIN;
    for (int t = w; t < ntile; t += 4) {
      int64_t sc[16];
      scores_i64(c, 32 * t, rterm, sqv, INV, sc);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (32 * t + 8 * (i >> 2) + 4 * half + (i & 3) <= mypos) mx = sc[i] > mx ? sc[i] : mx;
    }
    const int64_t o = __shfl_xor(mx, 32, 64);
    mx = o > mx ? o : mx;
  }
  if (half == 0) L.red_mx[w][l32] = mx;
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) mx = L.red_mx[k][l32] > mx ? L.red_mx[k][l32] : mx;
  mxd = (double)mx;
  // pass 2: sum of exp
  int64_t es = 0;
  for (int t = w; t < ntile; t += 4) {
    if (FAST) {
      double sc[16];
      if (32 * t + 31 <= firstpos) scores_f64<false>(c, 32 * t, rt32, fscale, mypos, sc);
      else scores_f64<true>(c, 32 * t, rt32, fscale, mypos, sc);
      int part = 0;   // 16 terms <= 2^24
#pragma unroll
      for (int i = 0; i < 16; ++i) part += exp_f64(L.T, mxd, sc[i]);
      es += part;
    } else {
      int64_t sc[16];
      scores_i64(c, 32 * t, rterm, sqv, INV, sc);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (32 * t + 8 * (i >> 2) + 4 * half + (i & 3) <= mypos) es += lut_exp(L.T, mx - sc[i]);
    }
  }
  es += __shfl_xor(es, 32, 64);
  if (half == 0) L.red_es[w][l32] = es;
  __syncthreads();
  es = L.red_es[0][l32] + L.red_es[1][l32] + L.red_es[2][l32] + L.red_es[3][l32];
  const double esd = (double)es, res = 1.0 / esd;
  // pass 3: p digits, then p . v per shift class
#pragma unroll
  for (int k = 0; k < NB + 2; ++k) acc[k] = v16i{};
  const int nsteps = (ntile + 3) / 4;
  for (int s = 0; s < nsteps; ++s) {
    const int t = 4 * s + w, buf = s & 1;
    v4i pa[3] = {v4i{}, v4i{}, v4i{}};
    if (t < ntile) {
      if (FAST) {
        double sc[16];
        if (32 * t + 31 <= firstpos) scores_f64<false>(c, 32 * t, rt32, fscale, mypos, sc);
        else scores_f64<true>(c, 32 * t, rt32, fscale, mypos, sc);
#pragma unroll
        for (int i = 0; i < 16; ++i) put_digits(pdiv_f64(exp_f64(L.T, mxd, sc[i]), esd, res), i, pa);
      } else {
        int64_t sc[16];
        scores_i64(c, 32 * t, rterm, sqv, INV, sc);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const bool ok = 32 * t + 8 * (i >> 2) + 4 * half + (i & 3) <= mypos;
          put_digits(ok ? (int)floordiv_rcp(shl64(lut_exp(L.T, mx - sc[i]), 20), es, res) : 0, i, pa);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pa[0][q] ^= 0x80808080;
        pa[1][q] ^= 0x80808080;
      }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) L.Pl[buf][w][a][lane] = pa[a];
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      if (4 * s + tt < ntile) {
        const int jb = 32 * (4 * s + tt);
        v4i pv[3], vb[NB];
#pragma unroll
        for (int a = 0; a < 3; ++a) pv[a] = L.Pl[buf][tt][a][lane];
#pragma unroll
        for (int b = 0; b < NB; ++b) vb[b] = *reinterpret_cast<const v4i*>(vd + b * vplane + jb);
#pragma unroll
        for (int a = 0; a < 3; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) acc[a + b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pv[a], vb[b], acc[a + b], 0, 0, 0);
      }
    }
  }
}

// grid (ceil(R / 32), H), block 256 (4 waves): query rows [32 x, 32 x + 32) of head y, heaviest tiles first.
// Key tiles of 32; in the first two passes wave w takes tiles w, w + 4, ...; in the third, each step of 4 tiles
// has wave w turn tile 4 step + w into p digits (LDS, double-buffered) and then every wave multiplies the 4
// tiles' p into V for its 32 dimensions. NB = V digits; the instantiation whose NB the KV head does not need
// returns at once (both are launched, so the host need not read vbits). Scores run in float64 when the block's
// shifts allow it exactly, else in int64.
template <int NB>
__global__ __launch_bounds__(256) void k_attn_fused(const int16_t* __restrict__ qq, const int32_t* __restrict__ sq,
                                                    const int8_t* __restrict__ kdig, const int32_t* __restrict__ ck,
                                                    const int32_t* __restrict__ skk, const int32_t* __restrict__ skmax,
                                                    const int8_t* __restrict__ vdig, const int32_t* __restrict__ vbits,
                                                    const int32_t* __restrict__ pos, const int32_t* __restrict__ Tg,
                                                    int64_t* __restrict__ out, int32_t* __restrict__ obits, int R, int H, int KV,
                                                    int nkeys, int kpad, int INV) {
  __shared__ int32_t T[EXACT_EXP_N];
  __shared__ v4i Pl[2][4][3][64];
  __shared__ int64_t red_mx[4][32], red_es[4][32];
  __shared__ int rowbits[32];
  const int h = blockIdx.y, kh = h / (H / KV);
  if ((vbits[kh] + 2 <= 32 ? 4 : 8) != NB) return;
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 32;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  for (int i = tid; i < EXACT_EXP_N; i += 256) T[i] = Tg[i];
  if (tid < 32) rowbits[tid] = 0;
  QK c;
  c.l32 = lane & 31;
  c.half = lane >> 5;
  c.kpad = kpad;
  c.kd = kdig + (int64_t)kh * 2 * 4 * kpad * 32;
  c.ckh = ck + (int64_t)kh * kpad;
  c.skh = skk + (int64_t)kh * kpad;
  const int qr = q0 + c.l32 < R ? q0 + c.l32 : R - 1;
  const int qlast = q0 + 31 < R ? q0 + 31 : R - 1;
  const int jmax = max(0, min(pos[qlast], nkeys - 1));       // positions increase with the row
  const int firstpos = max(0, min(pos[q0], nkeys - 1));
  const int mypos = max(0, min(pos[qr], nkeys - 1));
  const int ntile = jmax / 32 + 1;
  int sqs = 0;
  {
    const v4i* qp = reinterpret_cast<const v4i*>(qq + ((int64_t)qr * H + h) * AP_HD);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const v4i a0 = qp[(32 * kb + 16 * c.half) / 8], a1 = qp[(32 * kb + 16 * c.half) / 8 + 1];
      split_digits(a0, a1, c.qh[kb], c.ql[kb]);
      sqs += sum16(a0, a1);
    }
  }
  sqs += __shfl_xor(sqs, 32, 64);
  const int sqv = sq[(int64_t)qr * H + h];
  const bool fast = wave_max_i32(sqv) + skmax[kh] <= 33 && INV >= 0 && INV < (1 << 14);   // uniform over the block
  AttnLDS L{T, Pl, red_mx, red_es, rowbits};
  const int8_t* vd = vdig + (int64_t)kh * 8 * AP_HD * kpad + (int64_t)(32 * w + c.l32) * kpad + 16 * c.half;
  const int64_t vplane = (int64_t)AP_HD * kpad;
  v16i acc[NB + 2];
  if (fast) attn_body<NB, true>(c, L, 128 * (int64_t)sqs, sqv, INV, mypos, ntile, firstpos, vd, vplane, w, lane, acc);
  else attn_body<NB, false>(c, L, 128 * (int64_t)sqs, sqv, INV, mypos, ntile, firstpos, vd, vplane, w, lane, acc);
  // C layout: lane holds dimension 32 w + l32 of query rows 8 (i / 4) + 4 half + i % 4
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint64_t tot = 0;
#pragma unroll
    for (int k = 0; k < NB + 2; ++k) tot += (uint64_t)shl64((int64_t)acc[k][i], 8 * k);
    const int row = 8 * (i >> 2) + 4 * c.half + (i & 3);
    const int64_t o = shr64((int64_t)tot, 20);
    if (q0 + row < R) out[((int64_t)(q0 + row) * H + h) * AP_HD + 32 * w + c.l32] = o;
    atomicMax(rowbits + row, bitlen64(abs64(o)));
  }
  __syncthreads();
  if (obits && tid < 32 && q0 + tid < R) obits[(int64_t)(q0 + tid) * H + h] = rowbits[tid];
}

// workspace layout (bytes, each part 256-aligned): vdig KV*8*hd*kpad, kdig KV*2*hd*kpad, ck and skk KV*kpad*4
// each, vbits and skmax KV*4 each
static int64_t al256(int64_t n) { return (n + 255) & ~(int64_t)255; }
static int64_t ws_bytes(int KV, int kpad) {
  return al256((int64_t)KV * 8 * AP_HD * kpad) + al256((int64_t)KV * 2 * AP_HD * kpad) + 2 * al256((int64_t)KV * kpad * 4) +
         al256((int64_t)KV * 8);
}

}  // namespace exact

using namespace exact;

extern "C" int64_t exact_attention_prefill_workspace(int32_t KV, int32_t hd, int32_t nkeys) {
  if (KV <= 0 || hd != AP_HD || nkeys <= 0) return -1;
  return ws_bytes(KV, (nkeys + 31) / 32 * 32);
}

extern "C" int exact_attention_prefill(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                                       const int64_t* v, int32_t slot, const int32_t* pos, const int32_t* exp_t, int64_t* out,
                                       int32_t* obits, void* work, int64_t work_bytes, int32_t R, int32_t H, int32_t KV,
                                       int32_t hd, int32_t Smax, int32_t nkeys, int32_t INV, void* stream) {
  if (!qq || !sq || !kq || !sk || !v || !pos || !exp_t || !out || !work) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || slot < 0 || Smax <= 0 || nkeys <= 0 || nkeys > Smax) return EXACT_E_ARG;
  // per shift class, 3 digit pairs x nkeys products of |.| <= 2^14 stay below 2^31
  if (hd != AP_HD || nkeys > 32768) return EXACT_E_UNSUPPORTED;
  const int kpad = (nkeys + 31) / 32 * 32;
  if (work_bytes < ws_bytes(KV, kpad) || (reinterpret_cast<uintptr_t>(work) & 255)) return EXACT_E_ARG;
  int8_t* base = static_cast<int8_t*>(work);
  int8_t* vdig = base;
  int8_t* kdig = vdig + al256((int64_t)KV * 8 * AP_HD * kpad);
  int32_t* ck = reinterpret_cast<int32_t*>(kdig + al256((int64_t)KV * 2 * AP_HD * kpad));
  int32_t* skk = reinterpret_cast<int32_t*>(reinterpret_cast<int8_t*>(ck) + al256((int64_t)KV * kpad * 4));
  int32_t* vbits = reinterpret_cast<int32_t*>(reinterpret_cast<int8_t*>(skk) + al256((int64_t)KV * kpad * 4));
  int32_t* skmax = vbits + KV;
  hipStream_t st = as_stream(stream);
  int e = zero_bytes(vbits, (int64_t)KV * 8, st);
  if (e) return e;
  hipLaunchKernelGGL(k_vdigits, dim3(kpad / 32, KV), dim3(256), 0, st, v, slot, KV, Smax, nkeys, kpad, vdig, vbits);
  hipLaunchKernelGGL(k_kdigits, dim3(kpad / 32, KV), dim3(256), 0, st, kq, sk, slot, KV, Smax, nkeys, kpad, kdig, ck, skk,
                     skmax);
  const dim3 grid((R + 31) / 32, H);
  hipLaunchKernelGGL(k_attn_fused<4>, grid, dim3(256), 0, st, qq, sq, kdig, ck, skk, skmax, vdig, vbits, pos, exp_t, out, obits,
                     R, H, KV, nkeys, kpad, INV);
  hipLaunchKernelGGL(k_attn_fused<8>, grid, dim3(256), 0, st, qq, sq, kdig, ck, skk, skmax, vdig, vbits, pos, exp_t, out, obits,
                     R, H, KV, nkeys, kpad, INV);
  return launch_status("attention_prefill");
}
