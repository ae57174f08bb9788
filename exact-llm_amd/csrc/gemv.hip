// Exact group-128 int8 GEMV / small-R linear on CDNA4 matrix cores (gfx950).
//
// One wave owns a 64-row block of outputs and a run of 128-wide groups. Per group it streams the
// block's 8 KiB weight tile (eight fully coalesced 1 KiB loads, 16 B per lane) and feeds it to
// v_mfma_i32_16x16x64_i8 as the B operand (lane = output row within a 16-row sub-tile, 16 k per
// lane). The A operand holds up to 16 activation rows. For int16 activations (abits 15) each row
// is split into int8 digits hi = x >> 8 and lo = (x & 255) - 128 (exact_torch.py:101-102), so
// acc = 256 * hi.W + lo.W + 128 * colsum(W); the colsum comes from one extra all-ones row of A in
// the lo pass, read back with a lane shuffle. Each group's exact int32 accumulator is multiplied
// by its int16 scale and summed in int64 (t = sum_g acc_g * M_g, SPEC.md:18) before the next
// group starts. Runs of groups from different waves of the same row block are combined with
// 64-bit integer atomics, which are exact in any order.
//
// Reference: gemv_g128_v2 (experiments/speed_fair_kaggle.py:662-685) computes the same
// out[n] = sum_g (sum_{k in g} x[k] * wT[n,k]) * Mg[n,g] for one int16 row.
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace exact {

__device__ __forceinline__ int sel4(v4i v, int i) {
  return i == 0 ? v[0] : (i == 1 ? v[1] : (i == 2 ? v[2] : v[3]));
}

// Split 16 int16 values (two 16-byte loads) into 16 hi bytes and 16 (lo - 128) bytes.
__device__ __forceinline__ void split_a16(v4i p0, v4i p1, v4i& hi, v4i& lo) {
  // p0 = x[0..8), p1 = x[8..16): dword d holds x[2d] (low half) and x[2d+1] (high half)
  hi[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x07050301u);
  hi[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x07050301u);
  hi[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x07050301u);
  hi[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x07050301u);
  lo[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x06040200u) ^ 0x80808080;
  lo[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x06040200u) ^ 0x80808080;
  lo[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x06040200u) ^ 0x80808080;
  lo[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x06040200u) ^ 0x80808080;
}

template <int ABITS>
__global__ __launch_bounds__(256) void k_gemv_g128(const void* __restrict__ xv, const int8_t* __restrict__ wp,
                                                   const int16_t* __restrict__ mp, int64_t* __restrict__ t, int R,
                                                   int N, int K, int G, int gpw, int nsplit, int use_atomic) {
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nbs = (N + 63) >> 6;
  if (task >= nbs * nsplit) return;
  const int nb = task / nsplit, sp = task - nb * nsplit;
  const int g0 = sp * gpw;
  const int g1 = min(G, g0 + gpw);
  const int row = lane & 15, c = lane >> 4;

  int64_t acc[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[q][v] = 0;

  const v4i zero = {0, 0, 0, 0};
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  const int rsel = R & 3, rlane = (lane & 15) + 16 * (R >> 2);

  for (int g = g0; g < g1; ++g) {
    const int8_t* tile = wp + ((size_t)nb * G + g) * 8192;
    v4i b[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        b[h][q] = *reinterpret_cast<const v4i*>(tile + (4 * h + c) * 1024 + (16 * q + row) * 16);

    v4i ahi[2], alo[2];
    const int kb = g * 128 + 16 * c;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (ABITS == 15) {
        if (row < R) {
          const int16_t* xp = reinterpret_cast<const int16_t*>(xv) + (size_t)row * K + kb + 64 * h;
          v4i p0 = *reinterpret_cast<const v4i*>(xp);
          v4i p1 = *reinterpret_cast<const v4i*>(xp + 8);
          split_a16(p0, p1, ahi[h], alo[h]);
        } else {
          ahi[h] = zero;
          alo[h] = (row == R) ? ones : zero;
        }
      } else {
        ahi[h] = (row < R) ? *reinterpret_cast<const v4i*>(reinterpret_cast<const int8_t*>(xv) + (size_t)row * K + kb + 64 * h)
                           : zero;
      }
    }

    const int16_t* ms = mp + ((size_t)nb * G + g) * 64;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4i chi = zero, clo = zero;
      chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[0], b[0][q], chi, 0, 0, 0);
      chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[1], b[1][q], chi, 0, 0, 0);
      if (ABITS == 15) {
        clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[0], b[0][q], clo, 0, 0, 0);
        clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[1], b[1][q], clo, 0, 0, 0);
      }
      const int64_t m = (int64_t)ms[16 * q + row];
      int cs = 0;
      if (ABITS == 15) cs = __shfl(sel4(clo, rsel), rlane, 64);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        int a = (ABITS == 15) ? (chi[v] << 8) + clo[v] + 128 * cs : chi[v];
        acc[q][v] += (int64_t)a * m;
      }
    }
  }

#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N) {
        int64_t* dst = t + (size_t)r * N + n;
        if (use_atomic)
          atomicAdd(reinterpret_cast<unsigned long long*>(dst), (unsigned long long)acc[q][v]);
        else
          *dst = acc[q][v];
      }
    }
  }
}

__global__ void k_zero16(uint4* __restrict__ p, int64_t n16) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}
__global__ void k_zero1(uint8_t* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0;
}

int zero_bytes(void* dst, int64_t nbytes, hipStream_t st) {
  if (nbytes <= 0) return EXACT_OK;
  uint8_t* p = reinterpret_cast<uint8_t*>(dst);
  if ((reinterpret_cast<uintptr_t>(p) & 15) == 0 && nbytes >= 16) {
    int64_t n16 = nbytes / 16;
    int blocks = (int)std::min<int64_t>(cdiv(n16, 256), 4096);
    hipLaunchKernelGGL(k_zero16, dim3(blocks), dim3(256), 0, st, reinterpret_cast<uint4*>(p), n16);
    p += n16 * 16;
    nbytes -= n16 * 16;
  }
  if (nbytes > 0) hipLaunchKernelGGL(k_zero1, dim3((unsigned)cdiv(nbytes, 256)), dim3(256), 0, st, p, nbytes);
  return launch_status("zero");
}

// Work split: enough waves to cover the chip (~2048), whole groups per wave.
static void gemv_split(int N, int G, int* gpw, int* nsplit) {
  const int64_t tiles = (int64_t)((N + 63) / 64) * G;
  int g = (int)(tiles / 2048);
  if (g < 1) g = 1;
  if (g > G) g = G;
  *gpw = g;
  *nsplit = (G + g - 1) / g;
}

int gemv_launch(const void* x, int abits, const int8_t* wp, const int16_t* mp, int64_t* t, int R, int N, int K,
                hipStream_t st, bool zero_first) {
  const int G = K / 128;
  int gpw, nsplit;
  gemv_split(N, G, &gpw, &nsplit);
  const int use_atomic = nsplit > 1;
  if (use_atomic && zero_first) {
    int e = zero_bytes(t, (int64_t)R * N * 8, st);
    if (e) return e;
  }
  const int tasks = ((N + 63) / 64) * nsplit;
  dim3 grid((tasks + 3) / 4), block(256);
  if (abits == 15)
    hipLaunchKernelGGL(k_gemv_g128<15>, grid, block, 0, st, x, wp, mp, t, R, N, K, G, gpw, nsplit, use_atomic);
  else
    hipLaunchKernelGGL(k_gemv_g128<7>, grid, block, 0, st, x, wp, mp, t, R, N, K, G, gpw, nsplit, use_atomic);
  return launch_status("gemv_g128");
}

static int check_linear(const void* x, int abits, const int8_t* wp, const int16_t* mp, int64_t* t, int R, int N, int K) {
  if (!x || !wp || !mp || !t || R <= 0 || N <= 0 || K <= 0) return EXACT_E_ARG;
  if (abits != 15 && abits != 7) return EXACT_E_UNSUPPORTED;
  if (K % 128) return EXACT_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(wp) & 15)) return EXACT_E_UNSUPPORTED;
  return EXACT_OK;
}

}  // namespace exact

using namespace exact;

extern "C" int exact_zero(void* dst, int64_t nbytes, void* stream) {
  if (!dst && nbytes > 0) return EXACT_E_ARG;
  return zero_bytes(dst, nbytes, as_stream(stream));
}

extern "C" int exact_gemv_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, int64_t* t, int32_t R,
                               int32_t N, int32_t K, void* stream) {
  int e = check_linear(x, abits, wp, mp, t, R, N, K);
  if (e) return e;
  const int rmax = abits == 15 ? 15 : 16;   // one A row is the all-ones colsum row in the A16 mode
  if (R > rmax) return EXACT_E_UNSUPPORTED;
  return gemv_launch(x, abits, wp, mp, t, R, N, K, as_stream(stream), true);
}

extern "C" int exact_gemm_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, int64_t* t, int32_t R,
                               int32_t N, int32_t K, void* stream) {
  int e = check_linear(x, abits, wp, mp, t, R, N, K);
  if (e) return e;
  const int chunk = abits == 15 ? 15 : 16;
  const size_t xrow = (size_t)K * (abits == 15 ? 2 : 1);
  hipStream_t st = as_stream(stream);
  e = zero_bytes(t, (int64_t)R * N * 8, st);
  if (e) return e;
  for (int r0 = 0; r0 < R; r0 += chunk) {
    const int rr = std::min(chunk, R - r0);
    e = gemv_launch(reinterpret_cast<const int8_t*>(x) + r0 * xrow, abits, wp, mp, t + (size_t)r0 * N, rr, N, K, st, false);
    if (e) return e;
  }
  return EXACT_OK;
}
