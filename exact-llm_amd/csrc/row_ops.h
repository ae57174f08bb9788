// Row kernels' bodies as block-level device functions (one block per row).
#pragma once
#include "exact_common.h"

namespace exact {

template <typename T>
__device__ __forceinline__ void store_q(void* xq, int64_t i, int64_t v) {
  reinterpret_cast<T*>(xq)[i] = (T)v;
}

// The int16 value v of row r, column i as the interleaved int8 digit rows the int16 GEMM takes:
// x8[2r][i] = v >> 8, x8[2r + 1][i] = (v & 255) - 128 (the digit split of exact_torch.py:101-102).
__device__ __forceinline__ void store_digits(int8_t* x8, int64_t r, int64_t K, int64_t i, int64_t v) {
  x8[2 * r * K + i] = (int8_t)(v >> 8);
  x8[(2 * r + 1) * K + i] = (int8_t)((v & 255) - 128);
}

// Scratch of one block-level row pass: one array per reduction (the single-barrier reductions need
// their own).
struct RowScratch {
  int a[16], c[16];
  int64_t b[16], d[16];
};

// numpy floor division a // b for any int64 a and b != 0, kept out of line: the lean row program below calls it
// only when its quotient estimate leaves the range it is exact in.
static __device__ __attribute__((noinline)) int64_t floordiv_general(int64_t a, int64_t b) {
  return b > 0 ? floordiv_pos(a, b) : floordiv64(a, b);
}

// 1 / b in float64 from the hardware reciprocal and two Newton steps (relative error far below 2^-40 for b >= 1);
// the callers correct every quotient estimate made with it exactly.
__device__ __forceinline__ double rcp_f64(double b) {
  double r = __builtin_amdgcn_rcp(b);
  double e = __builtin_fma(-b, r, 1.0);
  r = __builtin_fma(r, e, r);
  e = __builtin_fma(-b, r, 1.0);
  return __builtin_fma(r, e, r);
}

// Round-half-up arithmetic shift right by a block-uniform 1 <= n <= 63, with int64 wrap (= shr64 there).
__device__ __forceinline__ int64_t rsh_pos(int64_t a, int n) {
  return (int64_t)((uint64_t)a + (1ULL << (n - 1))) >> n;
}

// bit length of max |v| over values whose largest is vmax and smallest vmin (vmin <= 0 <= vmax)
__device__ __forceinline__ int bitlen_maxabs(int64_t vmax, int64_t vmin) {
  const int64_t a = abs64(vmin);
  return bitlen64(a > vmax ? a : vmax);
}

// Row r of: x = x_in (+ round_shift(res_t, 28 - res_s[r]) when res_t), then xq, s = qrow(irms(x, g), bits)
// (exact_llm.py:41-46, 100-106). Outputs, each optional: x_out (x; may be x_in itself when one block owns the row),
// clear (res_t's row zeroed, likewise), xl (row r's quantised values, int16, LDS or global), xq_out (the quantised
// row, int16 when bits > 7 else int8), x8 (xq's interleaved digit rows) and s_out. The nt threads of the block hold
// EPT elements each (element i in thread i % nt). A consumer GEMV runs this in every block, so it is written lean,
// from bounds the program itself fixes:
//   k = max(bitlen(max |x|) - 24, 0) leaves |shr(x, k)| <= 2^24, so the squares are int32 products;
//   den = isqrt(sum / D + 1) << k is within a factor sqrt(D) of every |x|, so y = floor((x << 16) / den) (also
//   for a wrapped x << 16) has |y| < 2^24: a float64 quotient estimate is off by at most one and one exact int64
//   remainder test each way corrects it (the general floor division runs when an estimate leaves that range, or
//   den is outside (0, 2^62]);
//   the shifts k, 16, 28 - res_s and the qrow shift are uniform over the block, so their branches are too; loads
//   use clamped indices and mask the values past D, so only the stores are guarded.
// The global loads of one row's pass (x_in, res_t and the gains, clamped indices), kept apart so that a consumer GEMV
// can issue them before its first weight tile: the pass's first use then waits for these loads only.
template <int EPT>
struct NormIn {
  int64_t v[EPT], gv[EPT], rv[EPT];
  int rs;   // res_s[r] when res_t is given
};

template <int EPT>
__device__ __forceinline__ void norm_load(NormIn<EPT>& in, int r, int nt, const int64_t* x_in, const int64_t* res_t,
                                          const int32_t* __restrict__ res_s, const int64_t* __restrict__ g, int D) {
  const int tid = threadIdx.x;
  const int64_t* xr = x_in + (int64_t)r * D;
  const int64_t* tr = res_t ? res_t + (int64_t)r * D : nullptr;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt < D ? tid + j * nt : D - 1;
    in.v[j] = xr[i];
    in.gv[j] = g[i];
    in.rv[j] = tr ? tr[i] : 0;
  }
  in.rs = tr ? res_s[r] : 0;
}

template <int EPT>
__device__ __forceinline__ void norm_qrow_in(NormIn<EPT>& in, int r, int nt, const int64_t* res_t, int bits, int D,
                                             int16_t* xl,
                                             int64_t* x_out, int64_t* clear, int32_t* __restrict__ s_out, void* xq_out,
                                             int8_t* x8, RowScratch& sc) {
  const int tid = threadIdx.x;
  const double rD = rcp_f64((double)D);   // off the critical path: ready before the sum of squares
  int64_t (&v)[EPT] = in.v;
  int64_t (&gv)[EPT] = in.gv;
  {
    const int64_t (&rv)[EPT] = in.rv;
    if (res_t) {
      const int sh = 28 - in.rs;
      if (sh > 0) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) v[j] = (int64_t)((uint64_t)v[j] + (uint64_t)rsh_pos(rv[j], sh));
      } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) v[j] = (int64_t)((uint64_t)v[j] + (uint64_t)shl64(rv[j], -sh));
      }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const bool inside = tid + j * nt < D;
      v[j] = inside ? v[j] : 0;
      gv[j] = inside ? gv[j] : 0;
    }
  }
  if (x_out || clear) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = tid + j * nt;
      if (i < D) {
        if (x_out) x_out[(int64_t)r * D + i] = v[j];
        if (clear) clear[(int64_t)r * D + i] = 0;
      }
    }
  }
  int64_t hi = 0, lo = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    hi = v[j] > hi ? v[j] : hi;
    lo = v[j] < lo ? v[j] : lo;
  }
  // the bit length m of max |x| and, for the case m <= 24 (k = 0), the sum of squares, in one reduction: a thread
  // whose own values exceed 2^24 adds 0 (the sum is then not used), so every partial stays below 2^61
  const int ml = bitlen_maxabs(hi, lo);
  uint64_t s0 = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) s0 += (uint64_t)((int64_t)(int)v[j] * (int)v[j]);
  int m = wave_max_i32(ml);
  int64_t ss = wave_sum64(ml <= 24 ? (int64_t)s0 : 0);
  if ((tid & 63) == 0) {
    sc.a[tid >> 6] = m;
    sc.b[tid >> 6] = ss;
  }
  __syncthreads();
  {
    const int nw = nt >> 6;
    uint64_t st = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      m = i < nw && sc.a[i] > m ? sc.a[i] : m;
      st += i < nw ? (uint64_t)sc.b[i] : 0;
    }
    ss = (int64_t)st;
  }
  const int k = m > 24 ? m - 24 : 0;
  if (k > 0) {   // block-uniform
    ss = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int xs = (int)rsh_pos(v[j], k);   // |xs| <= 2^24
      ss += (int64_t)xs * xs;
    }
    ss = block_sum64_1(ss, sc.d);
  }
  // 0 <= ss < 2^62 (squares of at most 2^48, D of at most 2^13)
  // ms = ss // D + 1 and rt = isqrt(ms): float64 estimates (a reciprocal prepared early, the hardware square root),
  // each corrected exactly; the scalar chain is short because it sits between two block reductions
  int64_t qm = (int64_t)((double)ss * rD), rm = ss - qm * D;
  while (rm < 0) { --qm; rm += D; }
  while (rm >= D) { ++qm; rm -= D; }
  const int64_t ms = qm + 1;
  int64_t rt = (int64_t)__builtin_amdgcn_sqrt((double)ms);
  while (rt > 0 && rt * rt > ms) --rt;
  while ((rt + 1) * (rt + 1) <= ms) ++rt;
  if (rt < 1) rt = 1;
  const int64_t den = shl64(rt, k);
  const bool fast = den > 0 && den <= (1LL << 62);
  const double rden = rcp_f64((double)den);
  int yq[EPT];
  bool bad = !fast;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int64_t a = shl64(v[j], EXACT_F);
    const double qd = __builtin_floor((double)a * rden);
    bad |= !(__builtin_fabs(qd) < 1073741824.0);
    int q = (int)qd;
    const int64_t rem = (int64_t)((uint64_t)a - (uint64_t)(int64_t)q * (uint64_t)den);
    q += (rem >= den ? 1 : 0) - (rem < 0 ? 1 : 0);
    yq[j] = q;
  }
  int64_t z[EPT];
  if (!bad) {
#pragma unroll
    for (int j = 0; j < EPT; ++j) z[j] = rsh_pos((int64_t)((uint64_t)(int64_t)yq[j] * (uint64_t)gv[j]), EXACT_F);
  } else {   // not reached at the model shapes; exact for any int64
#pragma unroll
    for (int j = 0; j < EPT; ++j)
      z[j] = rsh_pos((int64_t)((uint64_t)floordiv_general(shl64(v[j], EXACT_F), den) * (uint64_t)gv[j]), EXACT_F);
  }
  hi = 0;
  lo = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {   // gains past D are 0, so z is 0 there
    hi = z[j] > hi ? z[j] : hi;
    lo = z[j] < lo ? z[j] : lo;
  }
  const int m2 = block_max_i32(bitlen_maxabs(hi, lo), sc.c);
  const int q = m2 > bits ? m2 - bits : 0;
  const int64_t lim = (1LL << bits) - 1;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    int64_t w = q ? rsh_pos(z[j], q) : z[j];
    w = w > lim ? lim : (w < -lim ? -lim : w);
    const int i = tid + j * nt;
    if (i < D) {
      if (xl) xl[i] = (int16_t)w;
      if (xq_out) {
        if (bits <= 7) store_q<int8_t>(xq_out, (int64_t)r * D + i, w);
        else store_q<int16_t>(xq_out, (int64_t)r * D + i, w);
      }
      if (x8) store_digits(x8, r, D, i, w);
    }
  }
  if (tid == 0 && s_out) s_out[r] = q;
}

template <int EPT>
__device__ __forceinline__ void norm_qrow_row(int r, int nt, const int64_t* x_in, const int64_t* res_t,
                                              const int32_t* __restrict__ res_s, const int64_t* __restrict__ g, int bits,
                                              int D, int16_t* xl, int64_t* x_out, int64_t* clear, int32_t* __restrict__ s_out,
                                              void* xq_out, int8_t* x8, RowScratch& sc) {
  NormIn<EPT> in;
  norm_load<EPT>(in, r, nt, x_in, res_t, res_s, g, D);
  norm_qrow_in<EPT>(in, r, nt, res_t, bits, D, xl, x_out, clear, s_out, xq_out, x8, sc);
}

}  // namespace exact
