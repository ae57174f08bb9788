// Integer sampler on the device (sample_int, exact_llm.py:256-259):
//   a = shr(lg * tnum, 16); p = isoftmax_row(a) (Q20); cum = cumsum(p);
//   target = (u20 * cum[-1]) >> 20 with u20 = splitmix64(seed, step) >> 44;
//   token = searchsorted(cum, target, 'right') = #{i : cum[i] <= target}
// One workgroup of SAMPLE_THREADS per row. Wave w owns the contiguous span [w*span, (w+1)*span) of the
// row and walks it 64 lanes at a time (coalesced loads); the running prefix inside a wave comes from a
// lane scan, the prefix before a wave from a scan over the waves' span sums. Since p >= 0, cum is
// non-decreasing, so the token is the number of prefix sums <= target.
#include "exact_common.h"
#include "abi_util.h"

namespace exact {

#define SAMPLE_THREADS 1024

__device__ __forceinline__ int64_t wave_incl_scan64(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t w = __shfl_up(v, o, 64);
    if (lane >= o) v = (int64_t)((uint64_t)v + (uint64_t)w);
  }
  return v;
}

__global__ __launch_bounds__(SAMPLE_THREADS) void k_sample(const int64_t* __restrict__ lg, int V, uint64_t seed,
                                                          const int32_t* __restrict__ step, int64_t tnum,
                                                          const int32_t* __restrict__ T, int32_t* __restrict__ ids,
                                                          int64_t* __restrict__ p_out) {
  __shared__ int64_t red_a[16], red_b[16], red_c[16];
  __shared__ int64_t wsum[SAMPLE_THREADS / 64];
  __shared__ int64_t wcnt[SAMPLE_THREADS / 64];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nw = blockDim.x >> 6;
  const int64_t* row = lg + (int64_t)r * V;
  const int span = ((V + nw - 1) / nw + 63) / 64 * 64;
  const int b0 = w * span, b1 = b0 + span < V ? b0 + span : V;
  // pass 1: row max of a
  int64_t mx = INT64_MIN;
  for (int i = b0 + lane; i < b1; i += 64) {
    const int64_t a = shr64(row[i] * tnum, EXACT_F);
    mx = a > mx ? a : mx;
  }
  mx = block_max64(mx, red_a);
  // pass 2: the softmax denominator
  int64_t es = 0;
  for (int i = b0 + lane; i < b1; i += 64) es += lut_exp(T, mx - shr64(row[i] * tnum, EXACT_F));
  es = block_sum64(es, red_b);
  // pass 3: each wave's sum of p
  int64_t ps = 0;
  for (int i = b0 + lane; i < b1; i += 64) ps += floordiv_pos(shl64(lut_exp(T, mx - shr64(row[i] * tnum, EXACT_F)), 20), es);
  ps = wave_sum64(ps);
  if (lane == 0) wsum[w] = ps;
  __syncthreads();
  int64_t pre = 0, total = 0;
  for (int j = 0; j < nw; ++j) {
    if (j < w) pre += wsum[j];
    total += wsum[j];
  }
  const int64_t u = (int64_t)(splitmix64(seed, (uint64_t)(int64_t)step[r]) >> 44);
  const int64_t target = (u * total) >> 20;
  // pass 4: count the prefix sums <= target, 64 at a time
  int64_t cnt = 0, carry = pre;
  for (int base = b0; base < b1; base += 64) {
    const int i = base + lane;
    int64_t p = 0;
    if (i < b1) p = floordiv_pos(shl64(lut_exp(T, mx - shr64(row[i] * tnum, EXACT_F)), 20), es);
    if (p_out && i < b1) p_out[(int64_t)r * V + i] = p;
    const int64_t c = carry + wave_incl_scan64(p, lane);
    if (i < b1 && c <= target) ++cnt;
    carry = __shfl(c, 63, 64);
  }
  cnt = wave_sum64(cnt);
  if (lane == 0) wcnt[w] = cnt;
  __syncthreads();
  if (tid == 0) {
    int64_t tok = 0;
    for (int j = 0; j < nw; ++j) tok += wcnt[j];
    ids[r] = (int32_t)tok;
  }
}

}  // namespace exact

using namespace exact;

extern "C" int exact_sample(const int64_t* lg, int32_t R, int32_t V, uint64_t seed, const int32_t* step, int64_t tnum,
                            const int32_t* exp_t, int32_t* ids, int64_t* p_out, void* stream) {
  if (!lg || !step || !exp_t || !ids || R <= 0 || V <= 0 || tnum <= 0) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_sample, dim3(R), dim3(SAMPLE_THREADS), 0, as_stream(stream), lg, V, seed, step, tnum, exp_t, ids,
                     p_out);
  return launch_status("sample");
}
