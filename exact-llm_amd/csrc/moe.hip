// Mixture-of-experts routing, dispatch and combination (MoEInt.moe, moe_exact_kaggle.py:454-467).
//
//   logits = shr(t_router, 28 - s)                        router linear, no bias
//   p      = isoftmax(logits) over all experts (Q20)      exact_llm.py:109-115
//   sel    = the top-k experts by a stable sort of -p    ties go to the lower expert index
//   out    = sum_j shr(p_j * down_e(h_e), 20) + shr(isig(sgate(m)) * shared(m), 16)
//
// Dispatch groups the R x k (row, expert) pairs by expert (stable: row-major order inside an expert)
// and cuts each expert's pairs into chunks of at most chunk_rows, so the expert GEMV streams each
// expert's weights once per chunk instead of once per pair. The combination is exact in any order.
#include "exact_common.h"
#include "abi_util.h"

#ifndef MOE_WAVE_PATHS
#define MOE_WAVE_PATHS 1   // routers of at most 64 experts and at most 64 pairs: one-wave kernels
#endif

namespace exact {

// One block per row of t (row stride ld). The probabilities stay in LDS for the rank computation:
// expert i has rank #{j : p_j > p_i or (p_j == p_i and j < i)}, its position in a stable sort of -p.
// With gate_col >= 0 the same row also holds the shared expert's gate logit (the router and the gate
// linear share one GEMV): gate[r] = isig(shr(t[r][gate_col], 28 - s)).
__global__ void k_router_topk(int64_t* __restrict__ t, int ld, const int32_t* __restrict__ s, const int32_t* __restrict__ T,
                              int64_t* __restrict__ p_sel, int32_t* __restrict__ e_sel, int gate_col,
                              const int32_t* __restrict__ sig_t, int64_t* __restrict__ gate, int NE, int k, int clear_t) {
  extern __shared__ int64_t sp[];
  __shared__ int64_t red[16];
  const int r = blockIdx.x;
  const int sh = 28 - s[r];
  int64_t* tr = t + (int64_t)r * ld;
  if (gate_col >= 0 && threadIdx.x == 0) {
    gate[r] = lut16(sig_t, shr64(tr[gate_col], sh), true);
    if (clear_t) tr[gate_col] = 0;
  }
  int64_t mx = INT64_MIN;
  for (int i = threadIdx.x; i < NE; i += blockDim.x) {
    const int64_t y = shr64(tr[i], sh);
    if (clear_t) tr[i] = 0;
    sp[i] = y;
    mx = y > mx ? y : mx;
  }
  mx = block_max64(mx, red);
  int64_t es = 0;
  for (int i = threadIdx.x; i < NE; i += blockDim.x) es += lut_exp(T, mx - sp[i]);
  es = block_sum64(es, red);
  for (int i = threadIdx.x; i < NE; i += blockDim.x) sp[i] = floordiv_pos(shl64(lut_exp(T, mx - sp[i]), 20), es);
  __syncthreads();
  for (int i = threadIdx.x; i < NE; i += blockDim.x) {
    const int64_t pi = sp[i];
    int rank = 0;
    for (int j = 0; j < NE; ++j) {
      const int64_t pj = sp[j];
      rank += (pj > pi) || (pj == pi && j < i);
    }
    if (rank < k) {
      p_sel[(int64_t)r * k + rank] = pi;
      e_sel[(int64_t)r * k + rank] = i;
    }
  }
}

// Routers of at most 64 experts (decode rows): one wave per row, expert i in lane i. The same steps as k_router_topk
// with wave reductions, and the rank of lane i from the other lanes' probabilities read as scalars, one per step.
// Returns the lane's rank (k or more when not selected).
__device__ __forceinline__ int route_row_w(int64_t* __restrict__ t, int ld, const int32_t* __restrict__ s,
                                           const int32_t* __restrict__ T, int64_t* __restrict__ p_sel,
                                           int32_t* __restrict__ e_sel, int gate_col, const int32_t* __restrict__ sig_t,
                                           int64_t* __restrict__ gate, int NE, int k, int clear_t, int r, int lane) {
  const int sh = 28 - s[r];
  int64_t* tr = t + (int64_t)r * ld;
  if (gate_col >= 0 && lane == 0) {
    gate[r] = lut16(sig_t, shr64(tr[gate_col], sh), true);
    if (clear_t) tr[gate_col] = 0;
  }
  const bool in = lane < NE;
  const int64_t y = in ? shr64(tr[in ? lane : 0], sh) : INT64_MIN;
  if (in && clear_t) tr[lane] = 0;
  const int64_t mx = wave_max64(y);
  const int64_t e = in ? lut_exp(T, mx - y) : 0;
  const int64_t es = wave_sum64(e);
  const int64_t p = in ? floordiv_pos(shl64(e, 20), es) : -1;   // probabilities are >= 0: lanes past NE rank last
  int rank = 0;
  for (int j = 0; j < NE; ++j) {
    const int64_t pj = readlane64(p, j);
    rank += (pj > p) || (pj == p && j < lane);
  }
  if (!in) rank = k;
  if (rank < k) {
    p_sel[(int64_t)r * k + rank] = p;
    e_sel[(int64_t)r * k + rank] = lane;
  }
  return rank;
}

__global__ __launch_bounds__(64) void k_router_topk_w(int64_t* __restrict__ t, int ld, const int32_t* __restrict__ s,
                                                      const int32_t* __restrict__ T, int64_t* __restrict__ p_sel,
                                                      int32_t* __restrict__ e_sel, int gate_col, const int32_t* __restrict__ sig_t,
                                                      int64_t* __restrict__ gate, int NE, int k, int clear_t) {
  route_row_w(t, ld, s, T, p_sel, e_sel, gate_col, sig_t, gate, NE, k, clear_t, blockIdx.x, threadIdx.x);
}

// At most 64 pairs (decode rows): one wave, pair q in lane q (expert e, e past the pairs for lanes >= P). Its place in
// the stable order by (expert, q) counts the pairs before it; a pair whose index inside its expert is a multiple of CH
// starts a chunk, and the chunk's index counts the starts placed before it, which orders the chunks by expert and then
// position, as k_moe_dispatch does.
__device__ __forceinline__ void dispatch_w(int e, const int32_t* __restrict__ s, int32_t* __restrict__ pidx,
                                           int32_t* __restrict__ pair_row, int32_t* __restrict__ s_pair,
                                           int32_t* __restrict__ chunk_e, int32_t* __restrict__ chunk_p0,
                                           int32_t* __restrict__ chunk_n, int32_t* __restrict__ nchunks, int P, int k, int CH,
                                           int lane) {
  const bool in = lane < P;
  int pos = 0, first = 0, cnt = 0;
  for (int j = 0; j < P; ++j) {
    const int ej = __builtin_amdgcn_readlane(e, j);
    pos += (ej < e) || (ej == e && j < lane);
    first += ej < e;
    cnt += ej == e;
  }
  const int idx = pos - first;   // place inside the expert's pairs
  const bool start = in && idx % CH == 0;
  const uint64_t starts = __ballot(start);
  int cidx = 0;
  for (int j = 0; j < P; ++j) {
    const int pj = __builtin_amdgcn_readlane(pos, j);
    cidx += (int)((starts >> j) & 1) & (pj < pos ? 1 : 0);
  }
  if (in) {
    pidx[lane] = pos;
    pair_row[pos] = lane / k;
    s_pair[pos] = s[lane / k];
  }
  if (start) {
    chunk_e[cidx] = e;
    chunk_p0[cidx] = pos;
    chunk_n[cidx] = cnt - idx < CH ? cnt - idx : CH;
  }
  if (lane == 0) nchunks[0] = __popcll(starts);
}

__global__ __launch_bounds__(64) void k_moe_dispatch_w(const int32_t* __restrict__ e_sel, const int32_t* __restrict__ s,
                                                       int32_t* __restrict__ pidx, int32_t* __restrict__ pair_row,
                                                       int32_t* __restrict__ s_pair, int32_t* __restrict__ chunk_e,
                                                       int32_t* __restrict__ chunk_p0, int32_t* __restrict__ chunk_n,
                                                       int32_t* __restrict__ nchunks, int P, int k, int CH) {
  const int lane = threadIdx.x;
  const int e = lane < P ? e_sel[lane] : 0x7fffffff;
  dispatch_w(e, s, pidx, pair_row, s_pair, chunk_e, chunk_p0, chunk_n, nchunks, P, k, CH, lane);
}

// Decode rows (at most 64 experts, at most 64 pairs): the top-k of every row, then the dispatch of their pairs, in one
// wave; the selected experts reach the dispatch through LDS (pair r k + rank of row r is the lane of that rank).
__global__ __launch_bounds__(64) void k_moe_route_w(int64_t* __restrict__ t, int ld, const int32_t* __restrict__ s,
                                                    const int32_t* __restrict__ T, int64_t* __restrict__ p_sel,
                                                    int32_t* __restrict__ e_sel, int gate_col, const int32_t* __restrict__ sig_t,
                                                    int64_t* __restrict__ gate, int NE, int k, int clear_t, int R,
                                                    int32_t* __restrict__ pidx, int32_t* __restrict__ pair_row,
                                                    int32_t* __restrict__ s_pair, int32_t* __restrict__ chunk_e,
                                                    int32_t* __restrict__ chunk_p0, int32_t* __restrict__ chunk_n,
                                                    int32_t* __restrict__ nchunks, int CH) {
  __shared__ int32_t es[64];
  const int lane = threadIdx.x;
  for (int r = 0; r < R; ++r) {
    const int rank = route_row_w(t, ld, s, T, p_sel, e_sel, gate_col, sig_t, gate, NE, k, clear_t, r, lane);
    if (rank < k) es[r * k + rank] = lane;
  }
  __syncthreads();
  const int P = R * k;
  dispatch_w(lane < P ? es[lane] : 0x7fffffff, s, pidx, pair_row, s_pair, chunk_e, chunk_p0, chunk_n, nchunks, P, k, CH, lane);
}

// One block of 16 waves. Pair q = r * k + j. Wave w owns experts e = w, w + 16, ...: it walks the pairs 64 at a
// time, and a ballot of "pair q belongs to e" gives both the expert's count and, with the count of set bits
// below each lane, each pair's stable position (q order) inside its expert. Then the chunks of each expert.
// The pairs' expert ids are walked from registers, DISPATCH_RB blocks of 64 at a time, and the offsets come from
// a wave-level scan, so no step waits on a chain of LDS reads.
#define DISPATCH_RB 16
__global__ __launch_bounds__(1024) void k_moe_dispatch(const int32_t* __restrict__ e_sel, const int32_t* __restrict__ s,
                                                       int32_t* __restrict__ pidx, int32_t* __restrict__ pair_row,
                                                       int32_t* __restrict__ s_pair, int32_t* __restrict__ chunk_e,
                                                       int32_t* __restrict__ chunk_p0, int32_t* __restrict__ chunk_n,
                                                       int32_t* __restrict__ nchunks, int P, int NE, int k, int CH) {
  extern __shared__ int32_t lds[];
  int32_t* es = lds;              // P expert ids
  int32_t* cnt = es + P;          // NE counts
  int32_t* off = cnt + NE;        // NE pair offsets
  int32_t* coff = off + NE;       // NE chunk offsets
  int32_t* srow = coff + NE;      // P / k row shifts (no global load inside the pair walk)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int q = threadIdx.x; q < P; q += blockDim.x) es[q] = e_sel[q];
  for (int r = threadIdx.x; r < P / k; r += blockDim.x) srow[r] = s[r];
  for (int e = threadIdx.x; e < NE; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int b0 = 0; b0 < P; b0 += 64 * DISPATCH_RB) {
    int ev[DISPATCH_RB];
#pragma unroll
    for (int i = 0; i < DISPATCH_RB; ++i) {
      const int q = b0 + 64 * i + lane;
      ev[i] = q < P ? es[q] : -1;
    }
    const int nb = (P - b0 + 63) / 64 < DISPATCH_RB ? (P - b0 + 63) / 64 : DISPATCH_RB;   // blocks of 64 holding pairs
    for (int e = wave; e < NE; e += nw) {   // cnt[e] belongs to this wave
      int c = 0;
#pragma unroll
      for (int i = 0; i < DISPATCH_RB; ++i)
        if (i < nb) c += __popcll(__ballot(ev[i] == e));
      if (lane == 0) cnt[e] += c;
    }
  }
  __syncthreads();
  if (wave == 0) {   // exclusive scans of the counts and of the chunk counts, 64 experts at a time
    int po = 0, co = 0;
    for (int e0 = 0; e0 < NE; e0 += 64) {
      const int e = e0 + lane;
      const int c = e < NE ? cnt[e] : 0, nc = (c + CH - 1) / CH;
      int ic = c, inc = nc;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(ic, d, 64), un = __shfl_up(inc, d, 64);
        if (lane >= d) {
          ic += u;
          inc += un;
        }
      }
      if (e < NE) {
        off[e] = po + ic - c;
        coff[e] = co + inc - nc;
      }
      po += __shfl(ic, 63, 64);
      co += __shfl(inc, 63, 64);
    }
    if (lane == 0) nchunks[0] = co;
  }
  __syncthreads();
  const uint64_t below = lane ? (~0ULL >> (64 - lane)) : 0ULL;   // lanes below this one
  for (int e = wave; e < NE; e += nw) {
    const int n = cnt[e];
    for (int c = lane; c * CH < n; c += 64) {
      const int idx = coff[e] + c;
      chunk_e[idx] = e;
      chunk_p0[idx] = off[e] + c * CH;
      chunk_n[idx] = n - c * CH < CH ? n - c * CH : CH;
    }
  }
  for (int b0 = 0; b0 < P; b0 += 64 * DISPATCH_RB) {
    int ev[DISPATCH_RB];
#pragma unroll
    for (int i = 0; i < DISPATCH_RB; ++i) {
      const int q = b0 + 64 * i + lane;
      ev[i] = q < P ? es[q] : -1;
    }
    const int nb = (P - b0 + 63) / 64 < DISPATCH_RB ? (P - b0 + 63) / 64 : DISPATCH_RB;
    for (int e = wave; e < NE; e += nw) {
      int run = off[e];
#pragma unroll
      for (int i = 0; i < DISPATCH_RB; ++i) {
        if (i >= nb) break;
        const bool mine = ev[i] == e;
        const uint64_t m = __ballot(mine);
        if (mine) {
          const int q = b0 + 64 * i + lane;
          const int pos = run + __popcll(m & below);
          pidx[q] = pos;
          pair_row[pos] = q / k;
          s_pair[pos] = srow[q / k];
        }
        run += __popcll(m);
      }
      if (lane == 0) off[e] = run;   // the next register batch continues after these pairs
    }
  }
}

// grid (ceil(D / 256), R), one element per thread: x += sum_j shr(p_j * shr(t_ed[pair], 28 - sh_pair), 20)
//                                                     + shr(gate * shr(t_sd, 28 - sh_s), 16)
__global__ __launch_bounds__(256) void k_moe_combine(int64_t* __restrict__ x, int64_t* __restrict__ t_ed,
                                                     const int32_t* __restrict__ sh_pair, const int64_t* __restrict__ p_sel,
                                                     const int32_t* __restrict__ pidx, int64_t* __restrict__ t_sd,
                                                     const int32_t* __restrict__ sh_s, const int64_t* __restrict__ gate, int D,
                                                     int k, int clear_t) {
  const int r = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x;
  if (d >= D) return;
  int64_t acc = 0;
  for (int j = 0; j < k; ++j) {
    const int q = pidx[r * k + j];
    int64_t* te = t_ed + (int64_t)q * D + d;
    const int64_t y = shr64(*te, 28 - sh_pair[q]);
    if (clear_t) *te = 0;
    acc += shr64(p_sel[r * k + j] * y, 20);
  }
  if (t_sd) {
    int64_t* ts = t_sd + (int64_t)r * D + d;
    acc += shr64(gate[r] * shr64(*ts, 28 - sh_s[r]), 16);
    if (clear_t) *ts = 0;
  }
  x[(int64_t)r * D + d] += acc;
}

}  // namespace exact

using namespace exact;

extern "C" int exact_router_topk(int64_t* t, int32_t ld, const int32_t* s, const int32_t* exp_t, int64_t* p_sel,
                                 int32_t* e_sel, int32_t gate_col, const int32_t* sig_t, int64_t* gate, int32_t R, int32_t NE,
                                 int32_t k, int32_t clear_t, void* stream) {
  if (!t || !s || !exp_t || !p_sel || !e_sel || R <= 0 || NE <= 0 || k <= 0 || k > NE || ld < NE) return EXACT_E_ARG;
  if (gate_col >= 0 && (gate_col >= ld || (gate_col < NE) || !sig_t || !gate)) return EXACT_E_ARG;
  if (NE > 4096) return EXACT_E_UNSUPPORTED;
  if (MOE_WAVE_PATHS && NE <= 64) {
    hipLaunchKernelGGL(k_router_topk_w, dim3(R), dim3(64), 0, as_stream(stream), t, ld, s, exp_t, p_sel, e_sel, gate_col, sig_t,
                       gate, NE, k, clear_t);
    return launch_status("router_topk");
  }
  hipLaunchKernelGGL(k_router_topk, dim3(R), dim3(256), NE * sizeof(int64_t), as_stream(stream), t, ld, s, exp_t, p_sel, e_sel,
                     gate_col, sig_t, gate, NE, k, clear_t);
  return launch_status("router_topk");
}

extern "C" int exact_moe_dispatch(const int32_t* e_sel, const int32_t* s, int32_t* pidx, int32_t* pair_row, int32_t* s_pair,
                                  int32_t* chunk_e, int32_t* chunk_p0, int32_t* chunk_n, int32_t* nchunks, int32_t R,
                                  int32_t NE, int32_t k, int32_t chunk_rows, void* stream) {
  if (!e_sel || !s || !pidx || !pair_row || !s_pair || !chunk_e || !chunk_p0 || !chunk_n || !nchunks) return EXACT_E_ARG;
  if (R <= 0 || NE <= 0 || k <= 0 || k > NE || chunk_rows <= 0) return EXACT_E_ARG;
  const int64_t P = (int64_t)R * k;
  if (MOE_WAVE_PATHS && P <= 64) {
    hipLaunchKernelGGL(k_moe_dispatch_w, dim3(1), dim3(64), 0, as_stream(stream), e_sel, s, pidx, pair_row, s_pair, chunk_e,
                       chunk_p0, chunk_n, nchunks, (int)P, k, chunk_rows);
    return launch_status("moe_dispatch");
  }
  if (P + 3LL * NE + R > 16384) return EXACT_E_UNSUPPORTED;   // 64 KiB of LDS
  hipLaunchKernelGGL(k_moe_dispatch, dim3(1), dim3(1024), (size_t)(P + 3 * NE + R) * sizeof(int32_t), as_stream(stream), e_sel,
                     s, pidx, pair_row, s_pair, chunk_e, chunk_p0, chunk_n, nchunks, (int)P, NE, k, chunk_rows);
  return launch_status("moe_dispatch");
}

extern "C" int exact_moe_route(int64_t* t, int32_t ld, const int32_t* s, const int32_t* exp_t, int64_t* p_sel, int32_t* e_sel,
                               int32_t gate_col, const int32_t* sig_t, int64_t* gate, int32_t R, int32_t NE, int32_t k,
                               int32_t clear_t, int32_t* pidx, int32_t* pair_row, int32_t* s_pair, int32_t* chunk_e,
                               int32_t* chunk_p0, int32_t* chunk_n, int32_t* nchunks, int32_t chunk_rows, void* stream) {
  if (!t || !s || !exp_t || !p_sel || !e_sel || R <= 0 || NE <= 0 || k <= 0 || k > NE || ld < NE) return EXACT_E_ARG;
  if (gate_col >= 0 && (gate_col >= ld || (gate_col < NE) || !sig_t || !gate)) return EXACT_E_ARG;
  if (!pidx || !pair_row || !s_pair || !chunk_e || !chunk_p0 || !chunk_n || !nchunks || chunk_rows <= 0) return EXACT_E_ARG;
  if (NE > 64 || (int64_t)R * k > 64) return EXACT_E_UNSUPPORTED;   // one wave: an expert a lane, a pair a lane
  hipLaunchKernelGGL(k_moe_route_w, dim3(1), dim3(64), 0, as_stream(stream), t, ld, s, exp_t, p_sel, e_sel, gate_col, sig_t,
                     gate, NE, k, clear_t, R, pidx, pair_row, s_pair, chunk_e, chunk_p0, chunk_n, nchunks, chunk_rows);
  return launch_status("moe_route");
}

extern "C" int exact_moe_combine(int64_t* x, int64_t* t_ed, const int32_t* sh_pair, const int64_t* p_sel, const int32_t* pidx,
                                 int64_t* t_sd, const int32_t* sh_s, const int64_t* gate, int32_t R, int32_t D, int32_t k,
                                 int32_t clear_t, void* stream) {
  if (!x || !t_ed || !sh_pair || !p_sel || !pidx || R <= 0 || D <= 0 || k <= 0) return EXACT_E_ARG;
  if (t_sd && (!sh_s || !gate)) return EXACT_E_ARG;
  hipLaunchKernelGGL(k_moe_combine, dim3((D + 255) / 256, R), dim3(256), 0, as_stream(stream), x, t_ed, sh_pair, p_sel, pidx,
                     t_sd, sh_s, gate, D, k, clear_t);
  return launch_status("moe_combine");
}
