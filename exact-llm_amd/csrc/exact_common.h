// Integer primitives of the exact program, device side (gfx950).
// Every function reproduces numpy int64 semantics (two's-complement wrap; the library is built
// with -fwrapv), so results are bit-identical to the CPU definitions:
//   round_shift  exact_llm.py:25-34   (round half up; n <= 0 shifts left)
//   bitlen       exact_llm.py:35-40
//   floor div    numpy '//' (exact_llm.py:103,105,115)
//   isqrt        exact_llm.py:97-99   (exact floor sqrt)
//   LUT interpolation of EXP_T / SILU_T / SIG_T  exact_llm.py:112-113,119-121; moe_exact_kaggle.py:421-423
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define EXACT_F 16
#define EXACT_ONE (1LL << 16)
#define EXACT_EXP_N 10242     // 40*256 + 2 entries
#define EXACT_LUT16_N 8194    // 32*256 + 2 entries

// Packed-weight tile order. Tile (nb, g) holds output rows [64 nb, 64 nb + 64) x input group g (8 KiB).
// Group-major order ([g][nb]) puts the tiles that concurrently running waves read next to each other,
// so the whole GPU sweeps the weight matrix front to back like a linear stream.
#ifndef EXACT_TILE_GN
#define EXACT_TILE_GN 1
#endif

namespace exact {

__host__ __device__ __forceinline__ int64_t tile_index(int64_t nb, int64_t g, int64_t nbs, int64_t G) {
  return EXACT_TILE_GN ? g * nbs + nb : nb * G + g;
}

__device__ __forceinline__ int64_t shl64(int64_t a, int m) {
  return m >= 64 ? 0 : (int64_t)((uint64_t)a << m);
}

// numpy: (a + (1 << (n-1))) >> n for n > 0, a << -n otherwise; shifts >= 64 follow numpy's rules.
__device__ __forceinline__ int64_t shr64(int64_t a, int n) {
  if (n <= 0) return shl64(a, -n);
  uint64_t half = (n - 1) < 64 ? (1ULL << (n - 1)) : 0ULL;
  int64_t s = (int64_t)((uint64_t)a + half);
  if (n >= 64) return s < 0 ? -1 : 0;
  return s >> n;
}

__device__ __forceinline__ int bitlen64(int64_t m) { return m <= 0 ? 0 : 64 - __clzll(m); }

__device__ __forceinline__ int64_t abs64(int64_t a) { return a < 0 ? (int64_t)(0 - (uint64_t)a) : a; }

// floor division for b > 0 (numpy '//')
__device__ __forceinline__ int64_t floordiv64(int64_t a, int64_t b) {
  int64_t q = a / b;
  int64_t r = a - q * b;
  return (r != 0 && ((r < 0) != (b < 0))) ? q - 1 : q;
}

// floor(a / b) for b > 0: a float64 estimate of the quotient, then an exact integer correction of the
// remainder into [0, b). Exact for every int64 a (the estimate only bounds the number of correction
// steps: one or two whenever |a / b| < 2^50, which covers every use here). b <= 0 (a softmax sum of an exp table
// without a positive entry 0, say) gives 0 rather than a correction loop that would not end.
__device__ __forceinline__ int64_t floordiv_pos(int64_t a, int64_t b) {
  if (b <= 0) return 0;
  double qd = __builtin_floor((double)a / (double)b);
  qd = qd > 9.2e18 ? 9.2e18 : (qd < -9.2e18 ? -9.2e18 : qd);
  int64_t q = (int64_t)qd;
  int64_t r = (int64_t)((uint64_t)a - (uint64_t)q * (uint64_t)b);
  while (r < 0) { --q; r += b; }
  while (r >= b) { ++q; r -= b; }
  return q;
}

// floor(a / b) for b > 0 given rb ~ 1 / b (one reciprocal for many divisions by the same b): the estimate is
// corrected exactly, as in floordiv_pos
__device__ __forceinline__ int64_t floordiv_rcp(int64_t a, int64_t b, double rb) {
  if (b <= 0) return 0;   // as floordiv_pos
  double qd = __builtin_floor((double)a * rb);
  qd = qd > 9.2e18 ? 9.2e18 : (qd < -9.2e18 ? -9.2e18 : qd);
  int64_t q = (int64_t)qd;
  int64_t r = (int64_t)((uint64_t)a - (uint64_t)q * (uint64_t)b);
  while (r < 0) { --q; r += b; }
  while (r >= b) { ++q; r -= b; }
  return q;
}

// SplitMix64 output for counter idx + 1 (Steele, Lea and Flood 2014; exact_llm.py:243-247)
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t key, uint64_t idx) {
  uint64_t z = key + (idx + 1ULL) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__device__ __forceinline__ int64_t isqrt64(int64_t n) {
  if (n <= 0) return 0;
  int64_t r = (int64_t)__builtin_sqrt((double)n);
  while (r > 0 && r * r > n) --r;
  while ((r + 1) * (r + 1) <= n) ++r;
  return r;
}

// exp LUT (Q24), d >= 0 for valid entries: e = T[i] - shr((T[i] - T[i+1]) * fr, 8)
__device__ __forceinline__ int64_t lut_exp(const int32_t* T, int64_t d) {
  int64_t i = d >> 8;
  if (i > EXACT_EXP_N - 2) i = EXACT_EXP_N - 2;
  int64_t fr = d & 255;
  int64_t a = T[i], b = T[i + 1];
  int64_t e = a - shr64((a - b) * fr, 8);
  return d < (40LL << EXACT_F) ? e : 0;
}

// SiLU (identity above 16) / sigmoid (1.0 above 16) tables on [-16, 16) at 1/256 steps
__device__ __forceinline__ int64_t lut16(const int32_t* T, int64_t x, bool sig) {
  if (x >= (16LL << EXACT_F)) return sig ? EXACT_ONE : x;
  if (x < -(16LL << EXACT_F)) return 0;
  int64_t t = x + (16LL << EXACT_F);
  int64_t i = t >> 8, fr = t & 255;
  int64_t a = T[i], b = T[i + 1];
  return a + shr64((b - a) * fr, 8);
}

// ---- wave (64-lane) reductions, for waves with every lane active. Within each row of 16 lanes four DPP steps
// (exchange with lane ^ 1, lane ^ 2, the mirrored lane of the 8-lane half row, the mirrored lane of the row) leave
// the row's result in all 16 lanes; the four row results are then read out of lanes 0, 16, 32, 48 into scalar
// registers, so the result is wave-uniform. (VALU-rate data movement instead of LDS-crossbar shuffles.)
template <int CTRL>
__device__ __forceinline__ int dpp32(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ int64_t dpp64(int64_t v) {
  const int lo = dpp32<CTRL>((int)(uint32_t)(uint64_t)v), hi = dpp32<CTRL>((int)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((int)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int64_t max64(int64_t a, int64_t b) { return a > b ? a : b; }
__device__ __forceinline__ int64_t wave_max64(int64_t v) {
  v = max64(v, dpp64<0xB1>(v));
  v = max64(v, dpp64<0x4E>(v));
  v = max64(v, dpp64<0x141>(v));
  v = max64(v, dpp64<0x140>(v));
  return max64(max64(readlane64(v, 0), readlane64(v, 16)), max64(readlane64(v, 32), readlane64(v, 48)));
}
__device__ __forceinline__ int64_t wave_sum64(int64_t v) {   // modulo 2^64
  auto add = [](int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); };
  v = add(v, dpp64<0xB1>(v));
  v = add(v, dpp64<0x4E>(v));
  v = add(v, dpp64<0x141>(v));
  v = add(v, dpp64<0x140>(v));
  return add(add(readlane64(v, 0), readlane64(v, 16)), add(readlane64(v, 32), readlane64(v, 48)));
}

// block reductions for blockDim.x a multiple of 64 (<= 1024); scratch holds >= 16 int64
__device__ __forceinline__ int64_t block_max64(int64_t v, int64_t* scratch) {
  v = wave_max64(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  int64_t r = scratch[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) r = i < nw && scratch[i] > r ? scratch[i] : r;
  return r;
}
__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t* scratch) {
  v = wave_sum64(v);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[w] = v;
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) r += i < nw ? (uint64_t)scratch[i] : 0;
  return (int64_t)r;
}

// Single-barrier block reductions: each call needs its own scratch array of 16 (no barrier protects a reused
// one).
__device__ __forceinline__ int64_t block_max64_1(int64_t v, int64_t* scratch) {
  v = wave_max64(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  const int nw = blockDim.x >> 6;
  int64_t r = scratch[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) r = i < nw && scratch[i] > r ? scratch[i] : r;
  return r;
}
// bitlen(max |v|) = max bitlen(|v|), so the max reductions of qrow / irms run on 32-bit bit lengths.
__device__ __forceinline__ int wave_max_i32(int v) {
  auto mx = [](int a, int b) { return a > b ? a : b; };
  v = mx(v, dpp32<0xB1>(v));
  v = mx(v, dpp32<0x4E>(v));
  v = mx(v, dpp32<0x141>(v));
  v = mx(v, dpp32<0x140>(v));
  return mx(mx(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
            mx(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int block_max_i32(int v, int* scratch) {
  v = wave_max_i32(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  const int nw = blockDim.x >> 6;
  int r = scratch[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) r = i < nw && scratch[i] > r ? scratch[i] : r;
  return r;
}
__device__ __forceinline__ int64_t block_sum64_1(int64_t v, int64_t* scratch) {
  v = wave_sum64(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  const int nw = blockDim.x >> 6;
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) r += i < nw ? (uint64_t)scratch[i] : 0;
  return (int64_t)r;
}

}  // namespace exact
