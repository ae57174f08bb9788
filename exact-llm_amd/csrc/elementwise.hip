// Integer nonlinearities and epilogues (one workgroup per row where a row reduction is needed).
// Each kernel restates one step of the reference's numeric program; see exact_common.h for the
// primitives and exact_hip.h for the reference line each entry point replaces.
#include "exact_common.h"
#include "abi_util.h"
#include "row_ops.h"

#include <mutex>

namespace exact {

static const char* g_err = "";
static char g_errbuf[256];
void set_error(const char* where, hipError_t e) {
  snprintf(g_errbuf, sizeof(g_errbuf), "%s: %s", where, hipGetErrorString(e));
  g_err = g_errbuf;
}

// qrow of a row held in `buf` (length K), writes xq / s for row r
__device__ __forceinline__ void qrow_store(const int64_t* buf, int K, int bits, void* xq, int32_t* s, int r,
                                           int64_t* red) {
  int64_t m = 0;
  for (int i = threadIdx.x; i < K; i += blockDim.x) {
    const int64_t a = abs64(buf[i]);
    m = a > m ? a : m;
  }
  m = block_max64(m, red);
  int sh = bitlen64(m) - bits;
  if (sh < 0) sh = 0;
  const int64_t lim = (1LL << bits) - 1;
  for (int i = threadIdx.x; i < K; i += blockDim.x) {
    int64_t q = shr64(buf[i], sh);
    q = q > lim ? lim : (q < -lim ? -lim : q);
    if (bits <= 7) store_q<int8_t>(xq, (int64_t)r * K + i, q);
    else store_q<int16_t>(xq, (int64_t)r * K + i, q);
  }
  if (threadIdx.x == 0) s[r] = sh;
}

// x (R, K) int64 -> qrow
__global__ void k_qrow(const int64_t* __restrict__ x, int bits, void* xq, int32_t* s, int K) {
  extern __shared__ int64_t buf[];
  __shared__ int64_t red[16];
  const int r = blockIdx.x;
  for (int i = threadIdx.x; i < K; i += blockDim.x) buf[i] = x[(int64_t)r * K + i];
  __syncthreads();
  qrow_store(buf, K, bits, xq, s, r, red);
}

// irms of one row, in place: exact_llm.py:100-106
__device__ void irms_inplace(int64_t* row, const int64_t* __restrict__ g, int D, int64_t* red) {
  int64_t m = 0;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const int64_t a = abs64(row[i]);
    m = a > m ? a : m;
  }
  m = block_max64(m, red);
  int k = bitlen64(m) - 24;
  if (k < 0) k = 0;
  int64_t ss = 0;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const int64_t xs = shr64(row[i], k);
    ss = (int64_t)((uint64_t)ss + (uint64_t)(xs * xs));
  }
  ss = block_sum64(ss, red);
  const int64_t ms = floordiv64(ss, D) + 1;
  int64_t rt = isqrt64(ms);
  if (rt < 1) rt = 1;
  const int64_t den = shl64(rt, k);
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const int64_t y = floordiv_pos(shl64(row[i], EXACT_F), den);
    row[i] = shr64(y * g[i], EXACT_F);
  }
  __syncthreads();
}

__global__ void k_irms(const int64_t* __restrict__ x, const int64_t* __restrict__ g, int64_t* __restrict__ y, int D) {
  extern __shared__ int64_t buf[];
  __shared__ int64_t red[16];
  const int r = blockIdx.x;
  for (int i = threadIdx.x; i < D; i += blockDim.x) buf[i] = x[(int64_t)r * D + i];
  __syncthreads();
  irms_inplace(buf, g, D, red);
  for (int i = threadIdx.x; i < D; i += blockDim.x) y[(int64_t)r * D + i] = buf[i];
}

// One workgroup per row, EPT elements per thread held in registers: every global load of the row
// (x, the residual total and the gains) is issued before the first use, so the row costs one memory
// round trip instead of one per loop iteration. x += rs(res_t, 28 - res_s) in place; then
// qrow(irms(x, g), bits) (exact_llm.py:41-46, 100-106).
template <int EPT>
__global__ __launch_bounds__(1024) void k_rmsnorm_qrow(int64_t* __restrict__ x, int64_t* __restrict__ res_t,
                                                       const int32_t* __restrict__ res_s, const int64_t* __restrict__ g,
                                                       int bits, void* xq, int32_t* s, int D, int clear_t, int8_t* x8) {
  __shared__ RowScratch sc;
  // one block per row: x is updated in place and the residual row cleared (each thread writes only what it read)
  norm_qrow_row<EPT>(blockIdx.x, blockDim.x, x, res_t, res_s, g, bits, D, nullptr, res_t ? x : nullptr,
                     (res_t && clear_t) ? res_t : nullptr, s, xq, x8, sc);
}

// Rows too long for one workgroup are split into slices of QSLICE elements; the producer kernel writes
// each slice's bit length of max |v| to part[r * nparts + slice], and k_quant_rows quantises every slice
// with the row's shift s = max(bitlen(max_row |v|) - bits, 0) (qrow, exact_llm.py:41-46), using
// bitlen(max |v|) = max bitlen(|v|).
#define QSLICE 1024

// gate|up total -> h = shr(isilu(g) * u, 16) (stored in hout (R, I) when given, else over the gate half),
// slice maxima of |h|
__global__ __launch_bounds__(256) void k_swiglu_part(int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                                     const int32_t* __restrict__ silu, int32_t* __restrict__ part, int I,
                                                     int nparts, int clear_t, int64_t* __restrict__ hout) {
  constexpr int EPT = QSLICE / 256;
  __shared__ int red[16];
  const int r = blockIdx.y, b = blockIdx.x;
  int64_t* tr = t + (int64_t)r * 2 * I;
  const int sh = 28 - s[r];
  int64_t gv[EPT], uv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * QSLICE + j * 256 + threadIdx.x;
    gv[j] = i < I ? tr[i] : 0;
    uv[j] = i < I ? tr[I + i] : 0;
  }
  int m = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * QSLICE + j * 256 + threadIdx.x;
    if (i < I) {
      const int64_t hv = shr64(lut16(silu, shr64(gv[j], sh), false) * shr64(uv[j], sh), EXACT_F);
      if (hout) {
        hout[(int64_t)r * I + i] = hv;
        if (clear_t) { tr[i] = 0; tr[I + i] = 0; }
      } else {
        tr[i] = hv;
        if (clear_t) tr[I + i] = 0;
      }
      const int bl = bitlen64(abs64(hv));
      m = bl > m ? bl : m;
    }
  }
  m = block_max_i32(m, red);
  if (threadIdx.x == 0) part[(int64_t)r * nparts + b] = m;
}

// One workgroup (1024 threads) per row with EPT gate/up pairs per thread in registers: all loads of the
// row are issued before the first use, one block reduction gives the row's shift, and the quantised
// row is stored directly (rows longer than 8192 use the multi-block pair below, which is faster there).
template <int EPT>
__global__ __launch_bounds__(1024) void k_swiglu_qrow_row(int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                                          const int32_t* __restrict__ silu, int bits, void* xq,
                                                          int32_t* __restrict__ sq, int I, int clear_t, int8_t* x8) {
  __shared__ int red[16];
  const int r = blockIdx.x, tid = threadIdx.x, nt = blockDim.x;
  int64_t* tr = t + (int64_t)r * 2 * I;
  const int sh = 28 - s[r];
  int64_t hv[EPT], uv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    hv[j] = i < I ? tr[i] : 0;
    uv[j] = i < I ? tr[I + i] : 0;
  }
  int m = 0;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    if (i < I) {
      hv[j] = shr64(lut16(silu, shr64(hv[j], sh), false) * shr64(uv[j], sh), EXACT_F);
      if (clear_t) { tr[i] = 0; tr[I + i] = 0; }
      const int bl = bitlen64(abs64(hv[j]));
      m = bl > m ? bl : m;
    }
  }
  m = block_max_i32(m, red);
  int q = m - bits;
  if (q < 0) q = 0;
  const int64_t lim = (1LL << bits) - 1;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + j * nt;
    if (i < I) {
      int64_t v = shr64(hv[j], q);
      v = v > lim ? lim : (v < -lim ? -lim : v);
      if (bits <= 7) store_q<int8_t>(xq, (int64_t)r * I + i, v);
      else store_q<int16_t>(xq, (int64_t)r * I + i, v);
      if (x8) store_digits(x8, r, I, i, v);
    }
  }
  if (tid == 0) sq[r] = q;
}

// grid (slices, R): xq[r][i] = clip(shr(src[r * ld + i], s_r), +-(2^bits - 1)), s_r from the slice maxima
__global__ __launch_bounds__(256) void k_quant_rows(int64_t* __restrict__ src, int64_t ld, const int32_t* __restrict__ part,
                                                    int nparts, int bits, void* xq, int32_t* __restrict__ s, int K,
                                                    int clear, int8_t* x8, int64_t* __restrict__ zero, int64_t zero_n) {
  __shared__ int qs;
  const int r = blockIdx.y, b = blockIdx.x;
  for (int64_t i = ((int64_t)r * gridDim.x + b) * blockDim.x + threadIdx.x; i < zero_n;
       i += (int64_t)gridDim.x * gridDim.y * blockDim.x)
    zero[i] = 0;
  if (threadIdx.x < 64) {
    int m = 0;
    for (int i = threadIdx.x; i < nparts; i += 64) {
      const int v = part[(int64_t)r * nparts + i];
      m = v > m ? v : m;
    }
    m = wave_max_i32(m);
    if (threadIdx.x == 0) {
      const int q = m - bits;
      qs = q < 0 ? 0 : q;
    }
  }
  __syncthreads();
  const int q = qs;
  if (b == 0 && threadIdx.x == 0) s[r] = q;
  const int64_t lim = (1LL << bits) - 1;
  constexpr int EPT = QSLICE / 256;
  int64_t vv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * QSLICE + j * 256 + threadIdx.x;
    vv[j] = i < K ? src[(int64_t)r * ld + i] : 0;
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * QSLICE + j * 256 + threadIdx.x;
    if (i < K) {
      if (clear) src[(int64_t)r * ld + i] = 0;
      int64_t v = shr64(vv[j], q);
      v = v > lim ? lim : (v < -lim ? -lim : v);
      if (bits <= 7) store_q<int8_t>(xq, (int64_t)r * K + i, v);
      else store_q<int16_t>(xq, (int64_t)r * K + i, v);
      if (x8) store_digits(x8, r, K, i, v);
    }
  }
}

__global__ void k_requant_group(const int64_t* __restrict__ t, const int32_t* __restrict__ s,
                                const int64_t* __restrict__ b, int64_t* __restrict__ y, int R, int N) {
  const int64_t total = (int64_t)R * N;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int r = (int)(i / N);
    const int n = (int)(i - (int64_t)r * N);
    const int64_t v = shr64(t[i], 28 - s[r]);
    y[i] = b ? v + b[n] : v;
  }
}

__global__ void k_requant_channel(const int64_t* acc, const int32_t* __restrict__ s, const int64_t* __restrict__ M,
                                  int Mbits, const int64_t* __restrict__ b, int64_t* y, int N) {
  __shared__ int64_t red[16];
  const int r = blockIdx.x;
  const int64_t* ar = acc + (int64_t)r * N;
  int64_t m = 0;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    const int64_t a = abs64(ar[i]);
    m = a > m ? a : m;
  }
  m = block_max64(m, red);
  int drop = bitlen64(m) + Mbits - 62;
  if (drop < 0) drop = 0;
  const int sh = 28 - s[r] - drop;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    const int64_t v = shr64(shr64(ar[i], drop) * M[i], sh);
    y[(int64_t)r * N + i] = b ? v + b[i] : v;
  }
}

__global__ void k_lut(const int64_t* __restrict__ x, const int32_t* __restrict__ T, int64_t* __restrict__ y, int64_t n,
                      int sig) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    y[i] = lut16(T, x[i], sig != 0);
}

__global__ void k_isoftmax(const int64_t* __restrict__ sc, const int32_t* __restrict__ n_valid,
                           const int32_t* __restrict__ T, int64_t* __restrict__ p, int N) {
  __shared__ int64_t red[16];
  const int r = blockIdx.x;
  const int nv = n_valid ? n_valid[r] : N;
  const int64_t* row = sc + (int64_t)r * N;
  int64_t mx = INT64_MIN;
  for (int i = threadIdx.x; i < nv; i += blockDim.x) mx = row[i] > mx ? row[i] : mx;
  mx = block_max64(mx, red);
  int64_t es = 0;
  for (int i = threadIdx.x; i < nv; i += blockDim.x) es += lut_exp(T, mx - row[i]);
  es = block_sum64(es, red);
  for (int i = threadIdx.x; i < N; i += blockDim.x)
    p[(int64_t)r * N + i] = i < nv ? floordiv_pos(shl64(lut_exp(T, mx - row[i]), 20), es) : 0;
}

__global__ void k_embed(const int32_t* __restrict__ ids, const int32_t* __restrict__ emb, int64_t* __restrict__ x,
                        int D, int V) {
  const int r = blockIdx.x;
  int id = ids[r];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  for (int i = threadIdx.x; i < D; i += blockDim.x) x[(int64_t)r * D + i] = emb[(int64_t)id * D + i];
}

// logits = shr(t, 28 - s) over slices of LSLICE columns; each slice's first maximum (value, index)
// goes to part; k_argmax_parts picks the row's first maximum (exact_llm.py:267: np.argmax)
#define LSLICE 4096
#ifndef LOGITS_THREADS
#define LOGITS_THREADS 1024   // threads of one slice's block (LSLICE / LOGITS_THREADS logits each)
#endif
__device__ __forceinline__ void argmax_merge(int64_t& best, int& bidx, int64_t ov, int oi) {
  if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
}

template <int NT>
__global__ __launch_bounds__(NT) void k_logits_part(int64_t* t, const int32_t* __restrict__ s, int64_t* lg,
                                                    int64_t* __restrict__ part, int N, int nparts, int clear_t) {
  __shared__ int64_t bv[NT / 64];
  __shared__ int bi[NT / 64];
  const int r = blockIdx.y, b = blockIdx.x;
  const int sh = 28 - s[r];
  constexpr int EPT = LSLICE / NT;
  int64_t tv[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * LSLICE + j * NT + threadIdx.x;
    tv[j] = i < N ? t[(int64_t)r * N + i] : 0;
  }
  int64_t best = INT64_MIN;
  int bidx = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = b * LSLICE + j * NT + threadIdx.x;
    if (i < N) {
      const int64_t v = shr64(tv[j], sh);
      if (clear_t) t[(int64_t)r * N + i] = 0;
      if (lg) lg[(int64_t)r * N + i] = v;
      if (v > best) { best = v; bidx = i; }   // i increases per thread: keeps the first max
    }
  }
  for (int o = 32; o > 0; o >>= 1) argmax_merge(best, bidx, __shfl_xor(best, o, 64), __shfl_xor(bidx, o, 64));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { bv[w] = best; bi[w] = bidx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < (int)(blockDim.x >> 6); ++i) argmax_merge(best, bidx, bv[i], bi[i]);
    part[((int64_t)r * nparts + b) * 2] = best;
    part[((int64_t)r * nparts + b) * 2 + 1] = bidx;
  }
}

__global__ void k_argmax_parts(const int64_t* __restrict__ part, int nparts, int32_t* __restrict__ ids) {
  const int r = blockIdx.x;
  int64_t best = INT64_MIN;
  int bidx = 0x7fffffff;
  for (int i = threadIdx.x; i < nparts; i += 64)
    argmax_merge(best, bidx, part[((int64_t)r * nparts + i) * 2], (int)part[((int64_t)r * nparts + i) * 2 + 1]);
  for (int o = 32; o > 0; o >>= 1) argmax_merge(best, bidx, __shfl_xor(best, o, 64), __shfl_xor(bidx, o, 64));
  if (threadIdx.x == 0) ids[r] = bidx;
}

__global__ void k_advance(int32_t* pos, int R) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < R) pos[i] += 1;
}

static inline int blk_for(int n) { return n >= 2048 ? 1024 : 256; }

}  // namespace exact

using namespace exact;

extern "C" int exact_version(void) { return 100; }
extern "C" const char* exact_last_error(void) { return g_err; }

#define SMEM_ROW_MAX 8192    // int64 entries staged per row in LDS (64 KiB)

extern "C" int exact_qrow(const int64_t* x, int32_t bits, void* xq, int32_t* s, int32_t R, int32_t K, void* stream) {
  if (!x || !xq || !s || R <= 0 || K <= 0 || bits < 1 || bits > 15) return EXACT_E_ARG;
  if (K > SMEM_ROW_MAX) return EXACT_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_qrow, dim3(R), dim3(blk_for(K)), K * 8, as_stream(stream), x, bits, xq, s, K);
  return launch_status("qrow");
}

extern "C" int exact_irms(const int64_t* x, const int64_t* g, int64_t* y, int32_t R, int32_t D, void* stream) {
  if (!x || !g || !y || R <= 0 || D <= 0) return EXACT_E_ARG;
  if (D > SMEM_ROW_MAX) return EXACT_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_irms, dim3(R), dim3(blk_for(D)), D * 8, as_stream(stream), x, g, y, D);
  return launch_status("irms");
}

#ifndef RMS_MAX_THREADS
#define RMS_MAX_THREADS 512      // rows of 2049..4096: 8 waves (3584: 7.5 -> 6.8 us a row in a graph)
#endif
#ifndef RMS_LARGE_THREADS
#define RMS_LARGE_THREADS 768    // rows above 4096: 12 waves (14B decode 196 -> 202 tok/s)
#endif
#ifndef RMS_EXACT_EPT
#define RMS_EXACT_EPT 1   // 5, 6 or 7 values a thread where the row needs them, not 8 (3584 over 512 threads: 5.33 -> 5.06 us)
#endif
#ifndef RMS_SMALL_THREADS
#define RMS_SMALL_THREADS 512    // rows of up to 2048: fewer waves per reduction (0.5B decode 893 -> 918 tok/s)
#endif
extern "C" int exact_rmsnorm_qrow(int64_t* x, int64_t* res_t, const int32_t* res_s, const int64_t* g, int32_t bits,
                                  void* xq, int32_t* s, int32_t R, int32_t D, int32_t clear_t, int8_t* x8, void* stream) {
  if (!x || !g || !xq || !s || R <= 0 || D <= 0 || bits < 1 || bits > 15 || (res_t && !res_s)) return EXACT_E_ARG;
  if (x8 && bits < 8) return EXACT_E_ARG;   // digit rows are of int16 values
  if (D > SMEM_ROW_MAX) return EXACT_E_UNSUPPORTED;
  const int tmax = D <= 2048 ? RMS_SMALL_THREADS : (D > 4096 ? RMS_LARGE_THREADS : RMS_MAX_THREADS);
  int nt = D >= tmax ? tmax : ((D + 63) / 64) * 64;
  if ((D + nt - 1) / nt > 8) nt = 1024;   // the row kernel holds at most 8 values per thread
  const int ept = (D + nt - 1) / nt;
  hipStream_t st = as_stream(stream);
#define RMS_GO(E) hipLaunchKernelGGL(k_rmsnorm_qrow<E>, dim3(R), dim3(nt), 0, st, x, res_t, res_s, g, bits, xq, s, D, clear_t, x8)
  if (ept <= 1) RMS_GO(1);
  else if (ept <= 2) RMS_GO(2);
  else if (ept <= 4) RMS_GO(4);
  else if (RMS_EXACT_EPT && ept <= 5) RMS_GO(5);
  else if (RMS_EXACT_EPT && ept <= 6) RMS_GO(6);
  else if (RMS_EXACT_EPT && ept <= 7) RMS_GO(7);
  else RMS_GO(8);
#undef RMS_GO
  return launch_status("rmsnorm_qrow");
}

#ifndef SWG_SMALL_THREADS
#define SWG_SMALL_THREADS 1024   // rows of up to 2048
#endif
extern "C" int exact_swiglu_qrow(int64_t* t, const int32_t* s, const int32_t* silu_t, int32_t bits, void* xq, int32_t* sq,
                                 int32_t* part, int32_t R, int32_t I, int32_t clear_t, int64_t* h, int8_t* x8, void* stream) {
  if (!t || !s || !silu_t || !part || R <= 0 || I <= 0 || bits < 1 || bits > 15) return EXACT_E_ARG;
  if (h == t || (!xq && !h) || (xq && !sq) || (x8 && (!xq || bits < 8))) return EXACT_E_ARG;
  hipStream_t st = as_stream(stream);
  if (!xq) {   // h and the slice bit lengths only: the consumer quantises (exact_gemv_g128_qrow_acc)
    const int np = (I + QSLICE - 1) / QSLICE;
    hipLaunchKernelGGL(k_swiglu_part, dim3(np, R), dim3(256), 0, st, t, s, silu_t, part, I, np, clear_t, h);
    return launch_status("swiglu_qrow");
  }
  const int tmax = I <= 2048 ? SWG_SMALL_THREADS : 1024;
  const int nt = I >= tmax ? tmax : ((I + 63) / 64) * 64;
  const int ept = (I + nt - 1) / nt;
#define SWG_GO(E) hipLaunchKernelGGL(k_swiglu_qrow_row<E>, dim3(R), dim3(nt), 0, st, t, s, silu_t, bits, xq, sq, I, clear_t, x8)
  if (ept <= 8) {   // rows up to 8192: one workgroup; longer rows go faster over many workgroups
    if (ept <= 2) SWG_GO(2);
    else if (ept <= 4) SWG_GO(4);
    else SWG_GO(8);
    return launch_status("swiglu_qrow");
  }
#undef SWG_GO
  const int np = (I + QSLICE - 1) / QSLICE;
  hipLaunchKernelGGL(k_swiglu_part, dim3(np, R), dim3(256), 0, st, t, s, silu_t, part, I, np, clear_t, h);
  if (h)
    hipLaunchKernelGGL(k_quant_rows, dim3(np, R), dim3(256), 0, st, h, (int64_t)I, part, np, bits, xq, sq, I, 0, x8, nullptr,
                       (int64_t)0);
  else
    hipLaunchKernelGGL(k_quant_rows, dim3(np, R), dim3(256), 0, st, t, (int64_t)2 * I, part, np, bits, xq, sq, I, clear_t, x8,
                       nullptr, (int64_t)0);
  return launch_status("swiglu_qrow");
}

extern "C" int exact_quant_rows(int64_t* src, int64_t ld, const int32_t* part, int32_t nparts, int32_t bits, void* xq,
                                int32_t* s, int32_t R, int32_t K, int32_t clear, int8_t* x8, int64_t* zero, int64_t zero_n,
                                void* stream) {
  if (!src || !part || !xq || !s || R <= 0 || K <= 0 || ld < K || nparts <= 0 || bits < 1 || bits > 15) return EXACT_E_ARG;
  if (x8 && bits < 8) return EXACT_E_ARG;
  if (zero_n < 0 || (zero_n > 0 && !zero)) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_quant_rows, dim3((K + QSLICE - 1) / QSLICE, R), dim3(256), 0, as_stream(stream), src, ld, part, nparts,
                     bits, xq, s, K, clear, x8, zero, zero_n);
  return launch_status("quant_rows");
}

extern "C" int exact_requant_group(const int64_t* t, const int32_t* s, const int64_t* b, int64_t* y, int32_t R, int32_t N,
                                   void* stream) {
  if (!t || !s || !y || R <= 0 || N <= 0) return EXACT_E_ARG;
  const int64_t total = (int64_t)R * N;
  const int blocks = (int)std::min<int64_t>(cdiv(total, 256), 8192);
  hipLaunchKernelGGL(k_requant_group, dim3(blocks), dim3(256), 0, as_stream(stream), t, s, b, y, R, N);
  return launch_status("requant_group");
}

extern "C" int exact_requant_channel(const int64_t* acc, const int32_t* s, const int64_t* M, int32_t Mbits, const int64_t* b,
                                     int64_t* y, int32_t R, int32_t N, void* stream) {
  if (!acc || !s || !M || !y || R <= 0 || N <= 0 || Mbits < 0 || Mbits > 62) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_requant_channel, dim3(R), dim3(blk_for(N)), 0, as_stream(stream), acc, s, M, Mbits, b, y, N);
  return launch_status("requant_channel");
}

extern "C" int exact_isilu(const int64_t* x, const int32_t* silu_t, int64_t* y, int64_t n, void* stream) {
  if (!x || !silu_t || !y || n < 0) return EXACT_E_ARG;
  if (n == 0) return EXACT_OK;
  hipLaunchKernelGGL(k_lut, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 8192)), dim3(256), 0, as_stream(stream), x, silu_t, y,
                     n, 0);
  return launch_status("isilu");
}

extern "C" int exact_isig(const int64_t* x, const int32_t* sig_t, int64_t* y, int64_t n, void* stream) {
  if (!x || !sig_t || !y || n < 0) return EXACT_E_ARG;
  if (n == 0) return EXACT_OK;
  hipLaunchKernelGGL(k_lut, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 8192)), dim3(256), 0, as_stream(stream), x, sig_t, y,
                     n, 1);
  return launch_status("isig");
}

extern "C" int exact_isoftmax(const int64_t* sc, const int32_t* n_valid, const int32_t* exp_t, int64_t* p, int32_t R,
                              int32_t N, void* stream) {
  if (!sc || !exp_t || !p || R <= 0 || N <= 0) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_isoftmax, dim3(R), dim3(256), 0, as_stream(stream), sc, n_valid, exp_t, p, N);
  return launch_status("isoftmax");
}

extern "C" int exact_embed(const int32_t* ids, const int32_t* emb, int64_t* x, int32_t R, int32_t D, int32_t V,
                           void* stream) {
  if (!ids || !emb || !x || R <= 0 || D <= 0 || V <= 0) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_embed, dim3(R), dim3(256), 0, as_stream(stream), ids, emb, x, D, V);
  return launch_status("embed");
}

extern "C" int exact_logits_argmax(int64_t* t, const int32_t* s, int64_t* lg, int32_t* ids, int64_t* part, int32_t R,
                                   int32_t N, int32_t clear_t, void* stream) {
  if (!t || !s || !part || R <= 0 || N <= 0 || (clear_t && lg == t)) return EXACT_E_ARG;
  const int np = (N + LSLICE - 1) / LSLICE;
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(k_logits_part<LOGITS_THREADS>, dim3(np, R), dim3(LOGITS_THREADS), 0, st, t, s, lg, part, N, np, clear_t);
  if (ids) hipLaunchKernelGGL(k_argmax_parts, dim3(R), dim3(64), 0, st, part, np, ids);
  return launch_status("logits_argmax");
}

// ---- exact_logits_argmax without a workspace argument ---------------------------------------------------------
// The per-slice maxima live in `scratch`, a file-scope device array: each GPU the library runs on holds its own
// copy (256 KiB) until the process ends. Host code never passes `scratch` itself to a kernel (on the host that
// name is a stand-in, not a device address): the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, on the entry point's first call there, and kept per device.
#define LA_SCRATCH_ROWS 64
#define LA_SCRATCH_N (1 << 20)
#define LA_SCRATCH_WORDS (LA_SCRATCH_ROWS * (LA_SCRATCH_N / LSLICE) * 2)
static __device__ __align__(256) int64_t scratch[LA_SCRATCH_WORDS];

#define LA_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static int64_t* g_scratch_dev[LA_MAX_DEVICES];

static int scratch_for_current_device(int64_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("logits_argmax_noalloc: hipGetDevice", e);
    return EXACT_E_LAUNCH;
  }
  if (dev < 0 || dev >= LA_MAX_DEVICES) return EXACT_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("logits_argmax_noalloc: hipGetSymbolAddress(scratch)", e != hipSuccess ? e : hipErrorInvalidSymbol);
      return EXACT_E_LAUNCH;
    }
    g_scratch_dev[dev] = static_cast<int64_t*>(p);
  }
  *out = g_scratch_dev[dev];
  return EXACT_OK;
}

extern "C" int exact_logits_argmax_noalloc(int64_t* t, const int32_t* s, int64_t* lg, int32_t* ids, int32_t R, int32_t N,
                                           int32_t clear_t, void* stream) {
  if (!t || !s || R <= 0 || N <= 0 || (clear_t && lg == t)) return EXACT_E_ARG;
  if (R > LA_SCRATCH_ROWS || N > LA_SCRATCH_N) return EXACT_E_UNSUPPORTED;
  int64_t* part = nullptr;
  const int e = scratch_for_current_device(&part);
  if (e) return e;
  const int np = (N + LSLICE - 1) / LSLICE;   // every (row, slice) entry read below is written first by this call
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(k_logits_part<LOGITS_THREADS>, dim3(np, R), dim3(LOGITS_THREADS), 0, st, t, s, lg, part, N, np, clear_t);
  if (ids) hipLaunchKernelGGL(k_argmax_parts, dim3(R), dim3(64), 0, st, part, np, ids);
  return launch_status("logits_argmax_noalloc");
}

extern "C" int exact_advance(int32_t* pos, int32_t R, void* stream) {
  if (!pos || R <= 0) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_advance, dim3((R + 255) / 256), dim3(256), 0, as_stream(stream), pos, R);
  return launch_status("advance");
}
