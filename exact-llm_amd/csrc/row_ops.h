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
  int64_t b[16];
};

// Row r of: if res_t, x += round_shift(res_t, 28 - res_s[r]) (written back; res_t zeroed when clear_t);
// then xq, s = qrow(irms(x, g), bits) (exact_llm.py:41-46, 100-106); x8 (optional): xq's digit rows too. The block's threads hold EPT
// elements each (blockDim.x * EPT >= D); every load of the row is issued before the first use.
template <int EPT>
__device__ __forceinline__ void rmsnorm_qrow_row(int r, int64_t* __restrict__ x, int64_t* __restrict__ res_t,
                                                 const int32_t* __restrict__ res_s, const int64_t* __restrict__ g,
                                                 int bits, void* xq, int32_t* s, int D, int clear_t, RowScratch& sc,
                                                 int8_t* x8 = nullptr) {
  const int tid = threadIdx.x, nt = blockDim.x;
  int64_t* xr = x + (int64_t)r * D;
  int64_t* tr = res_t ? res_t + (int64_t)r * D : nullptr;
  int64_t v[EPT], gv[EPT], rv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    v[j] = 0; gv[j] = 0; rv[j] = 0;
    if (i < D) {
      v[j] = xr[i];
      gv[j] = g[i];
      if (tr) rv[j] = tr[i];
    }
  }
  int m = 0;   // max bit length of |x|
  const int sh = tr ? 28 - res_s[r] : 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    if (i < D) {
      if (tr) {
        v[j] = (int64_t)((uint64_t)v[j] + (uint64_t)shr64(rv[j], sh));
        xr[i] = v[j];
        if (clear_t) tr[i] = 0;
      }
      const int bl = bitlen64(abs64(v[j]));
      m = bl > m ? bl : m;
    }
  }
  m = block_max_i32(m, sc.a);
  int k = m - 24;
  if (k < 0) k = 0;
  int64_t ss = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int64_t xs = shr64(v[j], k);   // elements past D hold 0
    ss = (int64_t)((uint64_t)ss + (uint64_t)(xs * xs));
  }
  ss = block_sum64_1(ss, sc.b);
  const int64_t ms = floordiv_pos(ss, D) + 1;   // ss >= 0 (a sum of squares; wraps only past 2^63, as numpy)
  int64_t rt = isqrt64(ms);
  if (rt < 1) rt = 1;
  const int64_t den = shl64(rt, k);
  const double rden = 1.0 / (double)den;
  int m2 = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    v[j] = shr64(floordiv_rcp(shl64(v[j], EXACT_F), den, rden) * gv[j], EXACT_F);
    const int bl = bitlen64(abs64(v[j]));
    m2 = (tid + j * nt < D && bl > m2) ? bl : m2;
  }
  m2 = block_max_i32(m2, sc.c);
  int q = m2 - bits;
  if (q < 0) q = 0;
  const int64_t lim = (1LL << bits) - 1;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    if (i < D) {
      int64_t w = shr64(v[j], q);
      w = w > lim ? lim : (w < -lim ? -lim : w);
      if (bits <= 7) store_q<int8_t>(xq, (int64_t)r * D + i, w);
      else store_q<int16_t>(xq, (int64_t)r * D + i, w);
      if (x8) store_digits(x8, r, D, i, w);
    }
  }
  if (tid == 0) s[r] = q;
}

}  // namespace exact
