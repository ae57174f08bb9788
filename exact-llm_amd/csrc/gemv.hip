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
#include "row_ops.h"

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

#ifndef GEMV_A8_SELECT
#define GEMV_A8_SELECT 0
#endif

// Per-group operands of one wave: the 8 KiB weight tile (8 x 16 B per lane), the A-operand bytes of
// the x rows (A8: 2 x 16 B, A16: 4 x 16 B raw int16) and the four int16 scales of the lane's columns.
struct GroupRegs {
  v4i b[8];
  v4i xa[4];
  int m[4];
};

// Scales of one group. mh: the high plane of wide scales when WIDE: M = mh * 2^15 + mp, mp in [0, 2^15).
template <bool WIDE>
__device__ __forceinline__ void load_scales(GroupRegs& G_, const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                            size_t tile, int row) {
  const int16_t* ms = mp + tile * 64 + row;
#pragma unroll
  for (int q = 0; q < 4; ++q) G_.m[q] = ms[16 * q];
  if constexpr (WIDE) {   // a template parameter: a run-time branch here cost the int8 kernels 40 VGPRs
    const int16_t* hs = mh + tile * 64 + row;
#pragma unroll
    for (int q = 0; q < 4; ++q) G_.m[q] |= (int)hs[16 * q] << 15;
  }
}

// The group's 8 KiB weight tile.
template <bool NT>
__device__ __forceinline__ void load_tile(GroupRegs& G_, const int8_t* __restrict__ wp, size_t tile, int row, int c) {
  const v4i* tp = reinterpret_cast<const v4i*>(wp + tile * 8192 + c * 1024 + row * 16);
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const v4i* a = tp + (4 * h * 1024 + 16 * q * 16) / 16;
      G_.b[4 * h + q] = NT ? __builtin_nontemporal_load(a) : *a;
    }
}

// A-operand bytes of group g. xrow: this lane's activation row (any valid row when the lane's row is unused: the
// lane's A row is zeroed in compute_group, after the data has arrived; zeroing the registers here, while the loads
// are in flight, made the compiler wait for every outstanding load of the wave, the prefetched tile included).
// xrow may point into LDS (a wave's quantised slice, offset so that group g sits at g * 128).
template <int ABITS>
__device__ __forceinline__ void load_x(GroupRegs& G_, const int8_t* xrow, int g, int c) {
  const int kb = g * 128 + 16 * c;
  if (ABITS == 15) {
    const int16_t* xp = reinterpret_cast<const int16_t*>(xrow) + kb;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      G_.xa[2 * h] = *reinterpret_cast<const v4i*>(xp + 64 * h);
      G_.xa[2 * h + 1] = *reinterpret_cast<const v4i*>(xp + 64 * h + 8);
    }
  } else {
    const int8_t* xp = xrow + kb;
#pragma unroll
    for (int h = 0; h < 2; ++h) G_.xa[h] = *reinterpret_cast<const v4i*>(xp + 64 * h);
  }
}

// issue order: scales, activations, then the tile (waiting on the tile drains the group)
template <int ABITS, bool NT, bool WIDE>
__device__ __forceinline__ void load_group(GroupRegs& G_, const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                           const int16_t* __restrict__ mh, const int8_t* xrow, bool valid,
                                           size_t tile, int g, int row, int c) {
  load_scales<WIDE>(G_, mp, mh, tile, row);
  load_x<ABITS>(G_, xrow, g, c);
  load_tile<NT>(G_, wp, tile, row, c);
}

// CT: int16 rows without the all-ones row; the caller adds 128 colterm (sum_g colsum_g M_g) once instead, so
// all 16 A rows carry activations.
// valid: the lane's A row is an activation row (row < R); other rows are zero, except the all-ones row R.
// One int16 row (VR = 1, so R = 1): its hi digits, lo digits and (without CT) the all-ones row are A rows 0, 1 and 2 of
// one MFMA chain, so their products land in C rows 0, 1 and 2, the same lane's three values: half the matrix-core work
// of the two chains below and no lane exchange for the column sums.
#ifndef GEMV_R1_PACK
#define GEMV_R1_PACK 1
#endif
template <int ABITS, int VR, bool CT = false>
__device__ __forceinline__ void compute_group(const GroupRegs& G_, int64_t (&acc)[4][VR], int R, int row, int lane,
                                              bool valid) {
  const v4i zero = {0, 0, 0, 0};
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  if constexpr (ABITS == 15 && VR == 1 && GEMV_R1_PACK) {
    v4i a[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i hi, lo;
      split_a16(G_.xa[2 * h], G_.xa[2 * h + 1], hi, lo);
      a[h] = row == 0 ? hi : (row == 1 ? lo : ((!CT && row == 2) ? ones : zero));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4i cc = zero;
      cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[0], G_.b[q], cc, 0, 0, 0);
      cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[1], G_.b[4 + q], cc, 0, 0, 0);
      // lanes 0..15 hold C rows 0, 1, 2 of their column in cc[0..2]; the other lanes' rows are never stored
      const int av = (cc[0] << 8) + cc[1] + (CT ? 0 : 128 * cc[2]);
      acc[q][0] += (int64_t)av * (int64_t)G_.m[q];
    }
    return;
  }
  v4i ahi[2], alo[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (ABITS == 15) {
      split_a16(G_.xa[2 * h], G_.xa[2 * h + 1], ahi[h], alo[h]);
      if (!valid) {
        ahi[h] = zero;
        alo[h] = (!CT && row == R) ? ones : zero;   // all-ones row: colsum(W) in the lo pass
      }
    } else {
#if GEMV_A8_SELECT
      ahi[h] = valid ? G_.xa[h] : zero;
#else
      ahi[h] = G_.xa[h];   // A row i feeds only C row i: the rows of unused lanes are never stored
#endif
      alo[h] = zero;
    }
  }
  const int rsel = R & 3, rlane = (lane & 15) + 16 * (R >> 2);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v4i chi = zero, clo = zero;
    chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[0], G_.b[q], chi, 0, 0, 0);
    chi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[1], G_.b[4 + q], chi, 0, 0, 0);
    if (ABITS == 15) {
      clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[0], G_.b[q], clo, 0, 0, 0);
      clo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[1], G_.b[4 + q], clo, 0, 0, 0);
    }
    const int64_t m = (int64_t)G_.m[q];
    int cs = 0;
    if (ABITS == 15 && !CT) cs = __shfl(sel4(clo, rsel), rlane, 64);
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int a = (ABITS == 15) ? (chi[v] << 8) + clo[v] + 128 * cs : chi[v];
      acc[q][v] += (int64_t)a * m;
    }
  }
}

// The group loop of one wave over groups [g0, g1) of row block nb. The next group's loads are issued
// before the current group's matrix-core work and every load is unconditional inside the loop, so
// each wave keeps two tiles (16 KiB) in flight. With one row per lane (VR = 1) a scheduling fence keeps the next group's
// loads ahead of this group's products: without it the compiler, aiming at an occupancy a 16-wave block cannot use,
// sinks them below the products and each group waits for its own loads (A8 7B pass 1.394-1.436 -> 1.359-1.402 ms).
// At VR = 4 the second register set does not fit the 128 registers of a 1024-thread block (bs8 gate|up 27.5 -> 40 us).
#ifndef GEMV_SCHED_FENCE
#define GEMV_SCHED_FENCE 1
#endif
// pro: run after the first group's weight tile is in flight and before its activations are read (the
// quantising GEMV fills its LDS slice there). pre: issues the prologue's own global loads before that tile's, so
// that their first use waits for them alone (loads complete in issue order: issued after the tile, they made the
// prologue wait for the tile's HBM latency first). The first tile is loaded without a branch (a wave without groups
// loads a valid one and never uses it): a branch around it would make the wait counts after the join assume the
// path without it.
#ifndef GEMV_PRE_FIRST
#define GEMV_PRE_FIRST 1
#endif
struct NoPrologue {
  __device__ void operator()() const {}
};

template <int ABITS, bool NT, int VR, typename Pro = NoPrologue, bool CT = false, bool WIDE = false,
          typename Pre = NoPrologue>
__device__ __forceinline__ void gemv_groups(int64_t (&acc)[4][VR], const int8_t* __restrict__ wp,
                                            const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                            const int8_t* xrow, bool valid, int R, int nb, int nbs, int G,
                                            int g0, int g1, int row, int c, int lane, Pro pro = Pro(), Pre pre = Pre()) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int v = 0; v < VR; ++v) acc[q][v] = 0;
  GroupRegs ra, rb;
  if constexpr (__is_same(Pro, NoPrologue)) {
    if (g0 >= g1) return;
    load_group<ABITS, NT, WIDE>(ra, wp, mp, mh, xrow, valid, tile_index(nb, g0, nbs, G), g0, row, c);
  } else {   // the first tile in flight while the prologue runs (one call site: the prologue may be long)
    if (GEMV_PRE_FIRST) {
      pre();
      __builtin_amdgcn_sched_barrier(0);
      const int gl = g0 < G ? g0 : G - 1;
      load_scales<WIDE>(ra, mp, mh, tile_index(nb, gl, nbs, G), row);
      load_tile<NT>(ra, wp, tile_index(nb, gl, nbs, G), row, c);
      __builtin_amdgcn_sched_barrier(0);
    } else {
      if (g0 < g1) {
        load_scales<WIDE>(ra, mp, mh, tile_index(nb, g0, nbs, G), row);
        load_tile<NT>(ra, wp, tile_index(nb, g0, nbs, G), row, c);
      }
      pre();
    }
    pro();
    if (g0 >= g1) return;
    load_x<ABITS>(ra, xrow, g0, c);
  }
  int g = g0;
  for (; g + 2 < g1; g += 2) {
    load_group<ABITS, NT, WIDE>(rb, wp, mp, mh, xrow, valid, tile_index(nb, g + 1, nbs, G), g + 1, row, c);
    if (GEMV_SCHED_FENCE && VR == 1) __builtin_amdgcn_sched_barrier(0);
    compute_group<ABITS, VR, CT>(ra, acc, R, row, lane, valid);
    load_group<ABITS, NT, WIDE>(ra, wp, mp, mh, xrow, valid, tile_index(nb, g + 2, nbs, G), g + 2, row, c);
    if (GEMV_SCHED_FENCE && VR == 1) __builtin_amdgcn_sched_barrier(0);
    compute_group<ABITS, VR, CT>(rb, acc, R, row, lane, valid);
  }
  if (g + 1 < g1) {
    load_group<ABITS, NT, WIDE>(rb, wp, mp, mh, xrow, valid, tile_index(nb, g + 1, nbs, G), g + 1, row, c);
    compute_group<ABITS, VR, CT>(ra, acc, R, row, lane, valid);
    compute_group<ABITS, VR, CT>(rb, acc, R, row, lane, valid);
  } else {
    compute_group<ABITS, VR, CT>(ra, acc, R, row, lane, valid);
  }
}

// One wave per (64-row block nb, group range [g0, g1)); BW waves per block take consecutive tasks.
// Lane l holds output rows 4*(l/16) + v, v < VR (VR = 1, 2 or 4 covers R <= 1, 2 or 16).
// out_mode 0: plain store (the wave owns all groups of its rows), 1: 64-bit atomic add.
// CT (int16 rows): colterm[n] = sum_g colsum_g M_g given, 128 colterm added by the first split of each row block,
// so R may be 16.
template <int ABITS, bool NT, int VR, int BW, bool CT = false, bool WIDE = false>
// int16 rows, one row, 4-wave blocks (the lm_head): 3 waves a SIMD (at most 168 registers; 172 otherwise)
__global__ __launch_bounds__(64 * BW, (ABITS == 15 && VR == 1 && BW == 4) ? 3 : 1) void k_gemv_g128(const void* __restrict__ xv, const int8_t* __restrict__ wp,
                                                       const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                                       int64_t* __restrict__ t, int R, int N, int K, int G, int nsplit,
                                                       int out_mode, const int64_t* __restrict__ colterm) {
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * BW + (threadIdx.x >> 6);
  const int nbs = (N + 63) >> 6;
  if (task >= nbs * nsplit) return;
  const int nb = task / nsplit, sp = task - nb * nsplit;
  const int g0 = (int)(((int64_t)sp * G) / nsplit);
  const int g1 = (int)(((int64_t)(sp + 1) * G) / nsplit);
  const int row = lane & 15, c = lane >> 4;
  const size_t xbytes = (size_t)K * (ABITS == 15 ? 2 : 1);
  const int8_t* xrow = reinterpret_cast<const int8_t*>(xv) + (size_t)(row < R ? row : 0) * xbytes;

  int64_t acc[4][VR];
  gemv_groups<ABITS, NT, VR, NoPrologue, CT, WIDE>(acc, wp, mp, mh, xrow, row < R, R, nb, nbs, G, g0, g1, row, c, lane);

#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
    const int64_t ct = (CT && sp == 0 && n < N) ? 128 * colterm[n] : 0;
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N) {
        int64_t* dst = t + (size_t)r * N + n;
        if (CT) acc[q][v] += ct;
        if (out_mode)
          atomicAdd(reinterpret_cast<unsigned long long*>(dst), (unsigned long long)acc[q][v]);
        else
          *dst = acc[q][v];
      }
    }
  }
}

// int64 activations each lane loads per row in the quantising GEMV: a wave's slice holds up to 64 * XQ_LOADS columns
#ifndef XQ_LOADS
#define XQ_LOADS 8
#endif

// GEMV whose int16 / int8 activations are quantised from int64 rows on the fly (qrow, exact_llm.py:41-46): row r's
// shift is s = max(bitlen(max |x_r|) - abits, 0), with bitlen(max |x_r|) = max_i part[r * nparts + i] as the producer
// kernel wrote it (attention's per-head bit lengths, or SwiGLU's per-slice ones). Each wave quantises the columns of
// its own groups into LDS (xs[r][g0 * 128 ...g1 * 128), clipped to +-(2^abits - 1)) and runs the group loop on them;
// block 0 writes s_out. Replaces a k_quant_rows launch + GEMV pair. t += x.W (accumulate).
// block bid of the launch (the kernel below, or a launch that runs it beside another GEMV)
template <int ABITS, bool NT, int VR, bool WIDE, int PL>
__device__ __forceinline__ void g128_xq_body(const int64_t* __restrict__ xs, int64_t ldx, const int32_t* __restrict__ part,
                                             int nparts, const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                             const int16_t* __restrict__ mh, int64_t* __restrict__ t,
                                             int32_t* __restrict__ s_out, int R, int N, int K, int G, int nsplit, int gmax,
                                             int bid) {
  extern __shared__ __attribute__((aligned(16))) int8_t xlds[];
  constexpr int EB = ABITS == 15 ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int task = bid * 4 + wave;
  const int nbs = (N + 63) >> 6;
  if (task >= nbs * nsplit) return;   // no block-wide barrier below
  const int nb = task / nsplit, sp = task - nb * nsplit;
  const int g0 = (int)(((int64_t)sp * G) / nsplit);
  const int g1 = (int)(((int64_t)(sp + 1) * G) / nsplit);
  const int ncol = (g1 - g0) * 128;
  const int rowb = gmax * 128 * EB;                       // LDS bytes per row of a wave's slice
  int8_t* mine = xlds + (size_t)wave * R * rowb;
  // quantise this wave's columns of every row: the row's slice bit lengths and its values are loaded together (row 0's
  // before the first weight tile)
  int pw[PL];   // up to 64 PL slice bit lengths, all loads issued before the first use
  int64_t xv[XQ_LOADS];
  auto ldrow = [&](int r) {
#pragma unroll
    for (int k = 0; k < PL; ++k) pw[k] = lane + 64 * k < nparts ? part[(int64_t)r * nparts + lane + 64 * k] : 0;
    const int64_t* src = xs + (int64_t)r * ldx + (int64_t)g0 * 128;
#pragma unroll
    for (int j = 0; j < XQ_LOADS; ++j) xv[j] = lane + 64 * j < ncol ? src[lane + 64 * j] : 0;
  };
  auto qrow = [&](int r) {
    const int64_t lim = (1LL << ABITS) - 1;
    int pv = pw[0];
#pragma unroll
    for (int k = 1; k < PL; ++k) pv = pw[k] > pv ? pw[k] : pv;
    const int m = wave_max_i32(pv);
    const int sh = m - ABITS > 0 ? m - ABITS : 0;
    if (bid == 0 && wave == 0 && lane == 0) s_out[r] = sh;
#pragma unroll
    for (int j = 0; j < XQ_LOADS; ++j) {
      const int i = lane + 64 * j;
      if (i < ncol) {
        int64_t q = shr64(xv[j], sh);
        q = q > lim ? lim : (q < -lim ? -lim : q);
        if (ABITS == 15) reinterpret_cast<int16_t*>(mine + (size_t)r * rowb)[i] = (int16_t)q;
        else mine[(size_t)r * rowb + i] = (int8_t)q;
      }
    }
  };
  auto first = [&]() { ldrow(0); };   // R >= 1 (the host entries refuse R <= 0)
  auto quantise = [&]() {
    qrow(0);
    for (int r = 1; r < R; ++r) {
      ldrow(r);
      qrow(r);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done (wave-private region)
    __builtin_amdgcn_wave_barrier();
  };
  const int row = lane & 15, c = lane >> 4;
  // group g's columns sit at (g - g0) * 128 of the slice: offset the row base back by g0 * 128 elements
  const int8_t* xrow = mine + (size_t)(row < R ? row : 0) * rowb - (ptrdiff_t)g0 * 128 * EB;
  int64_t acc[4][VR];
  gemv_groups<ABITS, NT, VR, decltype(quantise), false, WIDE, decltype(first)>(acc, wp, mp, mh, xrow, row < R, R, nb, nbs, G,
                                                                              g0, g1, row, c, lane, quantise, first);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N) atomicAdd(reinterpret_cast<unsigned long long*>(t + (size_t)r * N + n), (unsigned long long)acc[q][v]);
    }
  }
}

template <int ABITS, bool NT, int VR, bool WIDE, int PL>
// one row (VR = 1): 3 waves a SIMD (at most 168 registers), which the row 0 loads ahead of the first tile had cost
// (down 3584 x 18944 at 2 waves: 14.9 -> 16.3 us)
__global__ __launch_bounds__(256, VR == 1 ? 3 : 1) void k_gemv_g128_xq(const int64_t* __restrict__ xs, int64_t ldx,
                                                      const int32_t* __restrict__ part, int nparts,
                                                      const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                      const int16_t* __restrict__ mh, int64_t* __restrict__ t,
                                                      int32_t* __restrict__ s_out, int R, int N, int K, int G, int nsplit,
                                                      int gmax, int64_t* __restrict__ zero, int64_t zero_n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < zero_n; i += (int64_t)gridDim.x * blockDim.x)
    zero[i] = 0;
  g128_xq_body<ABITS, NT, VR, WIDE, PL>(xs, ldx, part, nparts, wp, mp, mh, t, s_out, R, N, K, G, nsplit, gmax, blockIdx.x);
}

// Operands of group g for one wave of the gate|up GEMV below: slots j = 0, 1 are sub-tiles qb, qb + 1 of the gate
// tile tg, slots 2, 3 the same sub-tiles of the up tile tu (a sub-tile is the 16 rows at byte 256 q of each 1 KiB
// chunk of the 8 KiB tile).
// scales and weight sub-tiles of one group (X: the activations too, loaded between them)
template <bool NT, bool WIDE, bool X = true>
__device__ __forceinline__ void load_gu_group(GroupRegs& G_, const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                              const int16_t* __restrict__ mh, const int8_t* xrow, size_t tg, size_t tu,
                                              int qb, int g, int row, int c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const size_t o = (j < 2 ? tg : tu) * 64 + 16 * (qb + (j & 1)) + row;
    G_.m[j] = mp[o];
    if constexpr (WIDE) G_.m[j] |= (int)mh[o] << 15;
  }
  if constexpr (X) load_x<15>(G_, xrow, g, c);
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int8_t* base = wp + (j < 2 ? tg : tu) * 8192;
      const v4i* a = reinterpret_cast<const v4i*>(base + h * 4096 + c * 1024 + (qb + (j & 1)) * 256 + row * 16);
      G_.b[4 * h + j] = NT ? __builtin_nontemporal_load(a) : *a;
    }
}

// Gate|up GEMV with the SwiGLU as its epilogue (decode rows, R <= 8, int16 activations). The linear holds the gate rows
// [0, I) and the up rows [I, 2I), I a multiple of 64. A pair is 32 gate columns (sub-tiles qb, qb + 1 of a 64-row tile)
// with the matching up columns; block b owns pairs b * NPB .. + NPB with NPB * KS waves: wave w = (pair p = w % NPB,
// k part kp = w / NPB) runs the group loop over its share of the groups for the pair's gate and up sub-tiles, so one lane
// holds a gate total and the up total of the same column. The k parts combine in LDS (no atomics, no zero-filled
// totals); the kp = 0 waves store h = shr(isilu(shr(g, 28 - s)) * shr(u, 28 - s), F) (exact_llm.py:179, as
// k_swiglu_part) and each pair's bit length of max |h| per row in part[r * I / 32 + pair], which the quantising down
// GEMV reads. tout (optional, (R, 2I)) receives the gate|up totals. Small blocks (NPB 1, KS 2: 2 I / 32 waves of 64
// lanes) spread the waves over the CUs better than larger ones (7B bs1 decode: 4-wave blocks of 64 columns 2311 us a
// step, 2-wave blocks of 32 columns 2194-2218, against 2311 for the GEMV + SwiGLU launches).
// NE > 0: the input rows are normalised in the kernel's own prologue, as k_gemv_g128_norm (every block runs
// x = x_in + rs(res_t, 28 - res_s) and qrow(irms(x, gain), 15) for each row into LDS while its first weight tiles load,
// NE elements per thread; block 0 writes x to x_out and the row shifts to s_out), so one launch replaces
// exact_rmsnorm_qrow + the gate|up GEMV + the SwiGLU.
template <bool NT, int VR, int NPB, int KS, bool WIDE, int NE>
__device__ __forceinline__ void gu_swiglu_body(const int16_t* __restrict__ x, const int8_t* __restrict__ wp,
                                               const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                               const int32_t* __restrict__ s, const int32_t* __restrict__ silu,
                                               int64_t* __restrict__ hout, int32_t* __restrict__ part,
                                               int64_t* __restrict__ tout, int R, int I, int K, int G,
                                               const int64_t* __restrict__ x_in, int64_t* __restrict__ x_out,
                                               const int64_t* __restrict__ res_t, const int32_t* __restrict__ res_s,
                                               const int64_t* __restrict__ gain, int32_t* __restrict__ s_out, int bid,
                                               int nblk) {
  __shared__ int64_t cmb[KS > 1 ? (KS - 1) * NPB * 4 * VR * 64 : 1];
  __shared__ int pm[NPB][8];
  extern __shared__ __attribute__((aligned(16))) int8_t xlds[];   // NE > 0: R rows of K int16 values
  __shared__ RowScratch nsc;
  __shared__ int32_t s_lds[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = wave % NPB, kp = wave / NPB;
  const int pair = bid * NPB + p;   // 32 gate columns: sub-tiles qb, qb + 1 of 64-column tile nb
  const int nb = pair >> 1, qb = 2 * (pair & 1), nbs = (2 * I) >> 6, ub = I >> 6;
  const int g0 = (int)(((int64_t)kp * G) / KS), g1 = (int)(((int64_t)(kp + 1) * G) / KS);
  const int row = lane & 15, c = lane >> 4;
  const bool valid = row < R;
  const int8_t* xrow = NE > 0 ? reinterpret_cast<const int8_t*>(reinterpret_cast<const int16_t*>(xlds) + (valid ? row : 0) * K)
                              : reinterpret_cast<const int8_t*>(x + (size_t)(valid ? row : 0) * K);
  int64_t acc[4][VR];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < VR; ++v) acc[j][v] = 0;
  if (NE > 0 || g0 < g1) {   // two groups in flight, as gemv_groups
    GroupRegs ra, rb;
    auto ld = [&](GroupRegs& G_, int g) {
      load_gu_group<NT, WIDE>(G_, wp, mp, mh, xrow, tile_index(nb, g, nbs, G), tile_index(ub + nb, g, nbs, G), qb, g, row, c);
    };
    if constexpr (NE > 0) {   // the first tiles in flight while the block normalises the rows (every wave takes part)
      // (row 0's norm inputs are loaded first, as gemv_groups' pre)
      int16_t* xl = reinterpret_cast<int16_t*>(xlds);
      int r0 = 0;
      if (GEMV_PRE_FIRST) {
        NormIn<NE> in0;
        norm_load<NE>(in0, 0, blockDim.x, x_in, res_t, res_s, gain, K);
        __builtin_amdgcn_sched_barrier(0);
        const int gl = g0 < G ? g0 : G - 1;
        load_gu_group<NT, WIDE, false>(ra, wp, mp, mh, xrow, tile_index(nb, gl, nbs, G), tile_index(ub + nb, gl, nbs, G), qb,
                                       gl, row, c);
        __builtin_amdgcn_sched_barrier(0);
        norm_qrow_in<NE>(in0, 0, blockDim.x, res_t, 15, K, xl, bid == 0 ? x_out : nullptr, nullptr, s_lds, nullptr, nullptr,
                         nsc);
        r0 = 1;
      } else if (g0 < g1) {
        load_gu_group<NT, WIDE, false>(ra, wp, mp, mh, xrow, tile_index(nb, g0, nbs, G), tile_index(ub + nb, g0, nbs, G), qb,
                                       g0, row, c);
      }
      for (int r = r0; r < R; ++r)
        norm_qrow_row<NE>(r, blockDim.x, x_in, res_t, res_s, gain, 15, K, xl + (size_t)r * K, bid == 0 ? x_out : nullptr,
                          nullptr, s_lds, nullptr, nullptr, nsc);
      __syncthreads();
      if (bid == 0 && (int)threadIdx.x < R) s_out[threadIdx.x] = s_lds[threadIdx.x];
      if (g0 >= g1) goto combine;
      load_x<15>(ra, xrow, g0, c);
    } else {
      ld(ra, g0);
    }
    int g = g0;
    for (; g + 2 < g1; g += 2) {
      ld(rb, g + 1);
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
      ld(ra, g + 2);
      compute_group<15, VR>(rb, acc, R, row, lane, valid);
    }
    if (g + 1 < g1) {
      ld(rb, g + 1);
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
      compute_group<15, VR>(rb, acc, R, row, lane, valid);
    } else {
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
    }
  }
combine:
  if constexpr (KS > 1) {
    if (kp > 0)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < VR; ++v) cmb[((((kp - 1) * NPB + p) * 4 + j) * VR + v) * 64 + lane] = acc[j][v];
    __syncthreads();
    if (kp == 0)
#pragma unroll
      for (int k = 1; k < KS; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < VR; ++v) acc[j][v] += cmb[((((k - 1) * NPB + p) * 4 + j) * VR + v) * 64 + lane];
  }
  if (kp == 0) {
    // lane (row, c) holds activation row r = 4c + v of gate|up column row: rows below R <= 8 sit in the lanes of
    // c = 0 and 1; each row's bit length is the maximum over its 16 lanes
    int bl[VR];
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int r = 4 * c + v;
      bl[v] = 0;
      if (c < 2 && r < R) {
        const int sh = 28 - (NE > 0 ? s_lds[r] : s[r]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = nb * 64 + 16 * (qb + j) + row;
          const int64_t gt = acc[j][v], ut = acc[2 + j][v];
          const int64_t hv = shr64(lut16(silu, shr64(gt, sh), false) * shr64(ut, sh), EXACT_F);
          hout[(size_t)r * I + i] = hv;
          if (tout) {
            tout[(size_t)r * 2 * I + i] = gt;
            tout[(size_t)r * 2 * I + I + i] = ut;
          }
          const int b = bitlen64(abs64(hv));
          bl[v] = b > bl[v] ? b : bl[v];
        }
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const int other = __shfl_xor(bl[v], o, 64);
        bl[v] = other > bl[v] ? other : bl[v];
      }
    }
    if (row == 0 && c < 2)
#pragma unroll
      for (int v = 0; v < VR; ++v) pm[p][4 * c + v] = bl[v];
  }
  __syncthreads();
  if ((int)threadIdx.x < R * NPB) {   // one bit length per pair (32 columns) and row, whatever NPB
    const int r = threadIdx.x / NPB, q = threadIdx.x - r * NPB;
    part[(size_t)r * nblk * NPB + bid * NPB + q] = pm[q][r];
  }
}

template <bool NT, int VR, int NPB, int KS, bool WIDE, int NE = 0>
__global__ __launch_bounds__(64 * NPB * KS) void k_gemv_gu_swiglu(const int16_t* __restrict__ x, const int8_t* __restrict__ wp,
                                                             const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                                             const int32_t* __restrict__ s, const int32_t* __restrict__ silu,
                                                             int64_t* __restrict__ hout, int32_t* __restrict__ part,
                                                             int64_t* __restrict__ tout, int R, int I, int K, int G,
                                                             const int64_t* __restrict__ x_in = nullptr,
                                                             int64_t* __restrict__ x_out = nullptr,
                                                             const int64_t* __restrict__ res_t = nullptr,
                                                             const int32_t* __restrict__ res_s = nullptr,
                                                             const int64_t* __restrict__ gain = nullptr,
                                                             int32_t* __restrict__ s_out = nullptr) {
  gu_swiglu_body<NT, VR, NPB, KS, WIDE, NE>(x, wp, mp, mh, s, silu, hout, part, tout, R, I, K, G, x_in, x_out, res_t, res_s,
                                            gain, s_out, blockIdx.x, gridDim.x);
}

// GEMV whose int16 input rows are normalised in its own prologue (decode): every block recomputes, for each of its R
// rows, x = x_in + rs(res_t, 28 - res_s) (res_t optional) and qrow(irms(x, g), 15) over the whole row (three block
// reductions, exact_llm.py:41-46, 100-106) into LDS while each wave's first weight tile is in flight, then runs the
// group loop on the LDS row. Block 0 writes x to x_out (another buffer: the other blocks are still reading x_in), the
// row shifts to s_out and, when xq_out is given, the quantised rows. t += x.W (accumulate). Replaces an
// exact_rmsnorm_qrow launch + exact_gemv_g128_acc.
// BW waves per block (4, or 8 for wide rows: one block per CU reads the row once, and the weight tiles of its 8
// tasks load while it normalises)
// (one row, 4-wave blocks, up to 8 values a thread: 3 waves a SIMD, at most 168 registers; 172 otherwise)
template <bool NT, int VR, int EPT, bool WIDE, int BW = 4>
__global__ __launch_bounds__(64 * BW, (VR == 1 && BW == 4 && EPT <= 8) ? 3 : 1) void k_gemv_g128_norm(const int64_t* __restrict__ x_in, int64_t* __restrict__ x_out,
                                                        const int64_t* __restrict__ res_t, const int32_t* __restrict__ res_s,
                                                        const int64_t* __restrict__ gain, const int8_t* __restrict__ wp,
                                                        const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                                        int64_t* __restrict__ t, int32_t* __restrict__ s_out,
                                                        int16_t* __restrict__ xq_out, int R, int N, int K, int G, int nsplit) {
  extern __shared__ __attribute__((aligned(16))) int8_t xlds[];   // R rows of K quantised int16 values
  __shared__ RowScratch sc;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int task = blockIdx.x * BW + wave;
  const int nbs = (N + 63) >> 6;
  const bool writer = blockIdx.x == 0;
  int16_t* xl = reinterpret_cast<int16_t*>(xlds);
  NormIn<EPT> in0;   // row 0's inputs, loaded before the first weight tile
  auto first = [&]() { norm_load<EPT>(in0, 0, 64 * BW, x_in, res_t, res_s, gain, K); };
  auto norm = [&]() {   // block-wide: every wave of the block runs it, with or without a task
    norm_qrow_in<EPT>(in0, 0, 64 * BW, res_t, 15, K, xl, writer ? x_out : nullptr, nullptr, writer ? s_out : nullptr,
                      writer ? xq_out : nullptr, nullptr, sc);
    for (int r = 1; r < R; ++r)
      norm_qrow_row<EPT>(r, 64 * BW, x_in, res_t, res_s, gain, 15, K, xl + (size_t)r * K, writer ? x_out : nullptr, nullptr,
                         writer ? s_out : nullptr, writer ? xq_out : nullptr, nullptr, sc);
    __syncthreads();
  };
  // waves without a task run the prologue (its barriers need every wave of the block) through the same call
  const bool has = task < nbs * nsplit;
  const int nb = has ? task / nsplit : 0, sp = has ? task - nb * nsplit : 0;
  const int g0 = has ? (int)(((int64_t)sp * G) / nsplit) : 0;
  const int g1 = has ? (int)(((int64_t)(sp + 1) * G) / nsplit) : 0;
  const int row = lane & 15, c = lane >> 4;
  const int8_t* xrow = reinterpret_cast<const int8_t*>(xl + (size_t)(row < R ? row : 0) * K);
  int64_t acc[4][VR];
  gemv_groups<15, NT, VR, decltype(norm), false, WIDE, decltype(first)>(acc, wp, mp, mh, xrow, row < R, R, nb, nbs, G, g0, g1,
                                                                        row, c, lane, norm, first);
  if (!has) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N) atomicAdd(reinterpret_cast<unsigned long long*>(t + (size_t)r * N + n), (unsigned long long)acc[q][v]);
    }
  }
}

// Expert GEMV (MoE): task = (chunk, 64-row block, group split). Chunk ch holds pairs
// [chunk_p0, chunk_p0 + chunk_n) of expert chunk_e; pair p reads activation row row_map[p] (or p
// when row_map is null) and adds its result into output row p (t must hold zeros or a running total).
// Expert e's packed linear starts at wp + e * w_stride, mp + e * m_stride.
template <int ABITS, bool NT>
__global__ __launch_bounds__(256) void k_gemv_experts(const void* __restrict__ xv, const int32_t* __restrict__ row_map,
                                                      const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                      int64_t w_stride, int64_t m_stride, const int32_t* __restrict__ chunk_e,
                                                      const int32_t* __restrict__ chunk_p0, const int32_t* __restrict__ chunk_n,
                                                      const int32_t* __restrict__ nchunks, int64_t* __restrict__ t, int N,
                                                      int K, int G, int nsplit) {
  constexpr int RMAX = ABITS == 15 ? 15 : 16;
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nbs = (N + 63) >> 6;
  const int per_chunk = nbs * nsplit;
  const int ch = task / per_chunk;
  if (ch >= nchunks[0]) return;
  const int rest = task - ch * per_chunk;
  const int nb = rest / nsplit, sp = rest - nb * nsplit;
  const int g0 = (int)(((int64_t)sp * G) / nsplit);
  const int g1 = (int)(((int64_t)(sp + 1) * G) / nsplit);
  const int e = chunk_e[ch], p0 = chunk_p0[ch];
  int R = chunk_n[ch];
  R = R < RMAX ? R : RMAX;
  const int row = lane & 15, c = lane >> 4;
  const int pr = p0 + (row < R ? row : 0);
  const size_t xbytes = (size_t)K * (ABITS == 15 ? 2 : 1);
  const int8_t* xrow = reinterpret_cast<const int8_t*>(xv) + (size_t)(row_map ? row_map[pr] : pr) * xbytes;

  int64_t acc[4][4];
  gemv_groups<ABITS, NT, 4>(acc, wp + (size_t)e * w_stride, mp + (size_t)e * m_stride, nullptr, xrow, row < R, R, nb, nbs,
                            G, g0,
                            g1, row, c, lane);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N)
        atomicAdd(reinterpret_cast<unsigned long long*>(t + (size_t)(p0 + r) * N + n), (unsigned long long)acc[q][v]);
    }
  }
}

// The routed experts' gate|up GEMV with the SwiGLU as its epilogue (MoE decode, dispatched chunks of at most 4 pairs):
// block b takes 32 gate columns (and their up columns) of chunk b / (I / 32), KS waves splitting the groups, combined
// in LDS as in k_gemv_gu_swiglu. Pair p0 + r (r < chunk_n) reads activation row row_map[p0 + r] against expert
// chunk_e's linear (wp + e w_stride, mp + e m_stride: gate rows [0, I), up rows [I, 2I)) and stores
// h[p0 + r][n] = shr(isilu(shr(g, 28 - s_pair[p0 + r])) * shr(u, 28 - s_pair[p0 + r]), F) (moe_exact_kaggle.py:461-463,
// exact_llm.py:179) and part[(p0 + r) (I / 32) + b % (I / 32)] = bit length of max |h| over the 32 columns. Blocks past
// the dispatched chunks exit.
template <bool NT, int KS>
__device__ __forceinline__ void experts_swiglu_body(const int16_t* __restrict__ x, const int32_t* __restrict__ row_map,
                                                    const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                    int64_t w_stride, int64_t m_stride, const int32_t* __restrict__ chunk_e,
                                                    const int32_t* __restrict__ chunk_p0, const int32_t* __restrict__ chunk_n,
                                                    const int32_t* __restrict__ nchunks, const int32_t* __restrict__ s_pair,
                                                    const int32_t* __restrict__ silu, int64_t* __restrict__ hout,
                                                    int32_t* __restrict__ part, int I, int K, int G, int bid) {
  constexpr int VR = 4;
  __shared__ int64_t cmb[KS > 1 ? (KS - 1) * 4 * VR * 64 : 1];
  __shared__ int pm[VR];
  const int lane = threadIdx.x & 63, kp = threadIdx.x >> 6;
  const int npb = I / 32;
  const int ch = bid / npb, pb = bid - ch * npb;
  if (ch >= nchunks[0]) return;   // uniform over the block: before any barrier
  const int e = chunk_e[ch], p0 = chunk_p0[ch];
  const int R = chunk_n[ch] < VR ? chunk_n[ch] : VR;
  wp += (int64_t)e * w_stride;
  mp += (int64_t)e * m_stride;
  const int nb = pb >> 1, qb = 2 * (pb & 1), nbs = (2 * I) >> 6, ub = I >> 6;
  const int g0 = (int)(((int64_t)kp * G) / KS), g1 = (int)(((int64_t)(kp + 1) * G) / KS);
  const int row = lane & 15, c = lane >> 4;
  const bool valid = row < R;
  const int pr = p0 + (valid ? row : 0);
  const int8_t* xrow = reinterpret_cast<const int8_t*>(x + (size_t)(row_map ? row_map[pr] : pr) * K);
  int64_t acc[4][VR];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int v = 0; v < VR; ++v) acc[j][v] = 0;
  if (g0 < g1) {
    GroupRegs ra, rb;
    auto ld = [&](GroupRegs& G_, int g) {
      load_gu_group<NT, false>(G_, wp, mp, nullptr, xrow, tile_index(nb, g, nbs, G), tile_index(ub + nb, g, nbs, G), qb, g, row,
                               c);
    };
    ld(ra, g0);
    int g = g0;
    for (; g + 2 < g1; g += 2) {
      ld(rb, g + 1);
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
      ld(ra, g + 2);
      compute_group<15, VR>(rb, acc, R, row, lane, valid);
    }
    if (g + 1 < g1) {
      ld(rb, g + 1);
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
      compute_group<15, VR>(rb, acc, R, row, lane, valid);
    } else {
      compute_group<15, VR>(ra, acc, R, row, lane, valid);
    }
  }
  if constexpr (KS > 1) {
    if (kp > 0)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < VR; ++v) cmb[(((kp - 1) * 4 + j) * VR + v) * 64 + lane] = acc[j][v];
    __syncthreads();
    if (kp == 0)
#pragma unroll
      for (int k = 1; k < KS; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < VR; ++v) acc[j][v] += cmb[(((k - 1) * 4 + j) * VR + v) * 64 + lane];
  }
  if (kp == 0) {   // lane (row, c = 0) holds pair r = v's gate and up totals of column row of sub-tiles qb, qb + 1
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      int bl = 0;
      if (c == 0 && v < R) {
        const int sh = 28 - s_pair[p0 + v];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = nb * 64 + 16 * (qb + j) + row;
          const int64_t hv = shr64(lut16(silu, shr64(acc[j][v], sh), false) * shr64(acc[2 + j][v], sh), EXACT_F);
          hout[(size_t)(p0 + v) * I + i] = hv;
          const int b = bitlen64(abs64(hv));
          bl = b > bl ? b : bl;
        }
      }
      bl = wave_max_i32(bl);
      if (lane == 0) pm[v] = bl;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < R) part[(size_t)(p0 + threadIdx.x) * npb + pb] = pm[threadIdx.x];
}

template <bool NT, int KS>
__global__ __launch_bounds__(64 * KS) void k_gemv_experts_swiglu(const int16_t* __restrict__ x, const int32_t* __restrict__ row_map,
                                                            const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                            int64_t w_stride, int64_t m_stride,
                                                            const int32_t* __restrict__ chunk_e,
                                                            const int32_t* __restrict__ chunk_p0,
                                                            const int32_t* __restrict__ chunk_n,
                                                            const int32_t* __restrict__ nchunks,
                                                            const int32_t* __restrict__ s_pair, const int32_t* __restrict__ silu,
                                                            int64_t* __restrict__ hout, int32_t* __restrict__ part, int I,
                                                            int K, int G) {
  experts_swiglu_body<NT, KS>(x, row_map, wp, mp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, s_pair, silu, hout,
                              part, I, K, G, blockIdx.x);
}

// The routed experts' down GEMV quantising its int64 input rows itself (MoE decode, chunks of at most 4 pairs): task =
// (chunk, 64-row block, group split) as k_gemv_experts; pair p0 + r's row xs[p0 + r] (ldx apart) is quantised with
// s = max(bitlen(max |row|) - 15, 0), bitlen(max |row|) = max_i part[(p0 + r) nparts + i] (qrow, exact_llm.py:41-46),
// into the wave's LDS slice (as k_gemv_g128_xq); t[p0 + r] += q(row) . W_e (64-bit atomics), s_out[p0 + r] = s.
template <bool NT, int PL>
__device__ __forceinline__ void experts_xq_body(const int64_t* __restrict__ xs, int64_t ldx, const int32_t* __restrict__ part,
                                                int nparts, const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                int64_t w_stride, int64_t m_stride, const int32_t* __restrict__ chunk_e,
                                                const int32_t* __restrict__ chunk_p0, const int32_t* __restrict__ chunk_n,
                                                const int32_t* __restrict__ nchunks, int64_t* __restrict__ t,
                                                int32_t* __restrict__ s_out, int N, int K, int G, int nsplit, int gmax,
                                                int bid) {
  constexpr int VR = 4;
  extern __shared__ __attribute__((aligned(16))) int8_t xlds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int task = bid * 4 + wave;
  const int nbs = (N + 63) >> 6;
  const int per_chunk = nbs * nsplit;
  const int ch = task / per_chunk;
  if (ch >= nchunks[0]) return;   // no block-wide barrier below
  const int rest = task - ch * per_chunk;
  const int nb = rest / nsplit, sp = rest - nb * nsplit;
  const int g0 = (int)(((int64_t)sp * G) / nsplit);
  const int g1 = (int)(((int64_t)(sp + 1) * G) / nsplit);
  const int e = chunk_e[ch], p0 = chunk_p0[ch];
  const int R = chunk_n[ch] < VR ? chunk_n[ch] : VR;
  const int ncol = (g1 - g0) * 128;
  const int rowb = gmax * 128 * 2;
  int8_t* mine = xlds + (size_t)wave * VR * rowb;
  int pw[PL];
  int64_t xv[XQ_LOADS];
  auto ldrow = [&](int r) {
    const int p = p0 + r;
#pragma unroll
    for (int k = 0; k < PL; ++k) pw[k] = lane + 64 * k < nparts ? part[(int64_t)p * nparts + lane + 64 * k] : 0;
    const int64_t* src = xs + (int64_t)p * ldx + (int64_t)g0 * 128;
#pragma unroll
    for (int j = 0; j < XQ_LOADS; ++j) xv[j] = lane + 64 * j < ncol ? src[lane + 64 * j] : 0;
  };
  auto qrow = [&](int r) {
    const int64_t lim = (1LL << 15) - 1;
    const int p = p0 + r;
    int pv = pw[0];
#pragma unroll
    for (int k = 1; k < PL; ++k) pv = pw[k] > pv ? pw[k] : pv;
    const int m = wave_max_i32(pv);
    const int sh = m - 15 > 0 ? m - 15 : 0;
    if (nb == 0 && sp == 0 && lane == 0) s_out[p] = sh;
#pragma unroll
    for (int j = 0; j < XQ_LOADS; ++j) {
      const int i = lane + 64 * j;
      if (i < ncol) {
        int64_t q = shr64(xv[j], sh);
        q = q > lim ? lim : (q < -lim ? -lim : q);
        reinterpret_cast<int16_t*>(mine + (size_t)r * rowb)[i] = (int16_t)q;
      }
    }
  };
  auto first = [&]() {   // row 0's loads ahead of the first weight tile
    if (R > 0) ldrow(0);
  };
  auto quantise = [&]() {
    if (R > 0) qrow(0);
    for (int r = 1; r < R; ++r) {
      ldrow(r);
      qrow(r);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes are done (wave-private region)
    __builtin_amdgcn_wave_barrier();
  };
  const int row = lane & 15, c = lane >> 4;
  const int8_t* xrow = mine + (size_t)(row < R ? row : 0) * rowb - (ptrdiff_t)g0 * 128 * 2;
  int64_t acc[4][VR];
  gemv_groups<15, NT, VR, decltype(quantise), false, false, decltype(first)>(acc, wp + (size_t)e * w_stride,
                                                                             mp + (size_t)e * m_stride, nullptr, xrow, row < R,
                                                                             R, nb, nbs, G, g0, g1, row, c, lane, quantise,
                                                                             first);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nb * 64 + 16 * q + row;
#pragma unroll
    for (int v = 0; v < VR; ++v) {
      const int r = 4 * c + v;
      if (r < R && n < N)
        atomicAdd(reinterpret_cast<unsigned long long*>(t + (size_t)(p0 + r) * N + n), (unsigned long long)acc[q][v]);
    }
  }
}

template <bool NT, int PL>
__global__ __launch_bounds__(256) void k_gemv_experts_xq(const int64_t* __restrict__ xs, int64_t ldx,
                                                         const int32_t* __restrict__ part, int nparts,
                                                         const int8_t* __restrict__ wp, const int16_t* __restrict__ mp,
                                                         int64_t w_stride, int64_t m_stride, const int32_t* __restrict__ chunk_e,
                                                         const int32_t* __restrict__ chunk_p0, const int32_t* __restrict__ chunk_n,
                                                         const int32_t* __restrict__ nchunks, int64_t* __restrict__ t,
                                                         int32_t* __restrict__ s_out, int N, int K, int G, int nsplit, int gmax) {
  experts_xq_body<NT, PL>(xs, ldx, part, nparts, wp, mp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, t, s_out, N, K,
                          G, nsplit, gmax, blockIdx.x);
}

// The reference's exact::gemv on its own tensors (speed_fair_kaggle.py:686-702): one int16 row x (K,), the
// row-major int8 weight wT (N, K) and int64 group scales Mg (N, G); out[n] = sum_g (sum_{k in g} x[k] wT[n][k]) Mg[n][g]
// in int64 (wrapping like the reference's int64 sums). No repacking. A wave owns a range of K (4 KiB, or 2 KiB for long
// rows) and a run of rows; lane l handles the 16-byte chunks l, l + 64, ... of the range, so one load instruction reads
// 1 KiB of one weight row, and the lanes l / 8 = j of a chunk hold one 128-wide group. The lane's x digits
// (hi = x >> 8, lo = (x & 255) - 128) stay in registers for all its rows; per chunk three int8 dot products give the
// lane's part of 256 hi.w + lo.w + 128 sum(w) = x.w (exact_torch.py:101-102), which the lane multiplies by its
// group's scale (sum_g M_g sum_lanes a = sum_lanes M_g a: the per-group sums need no reduction of their own), and the
// wave sums the row's int64 partials once. Rows are loaded two ahead of the one being summed, into two register sets
// used in turn; the row loop is unrolled whole (RPW rows a wave, a template parameter) and no load sits behind a
// branch, so each row waits only for its own loads. (A row loop with a back edge made the compiler copy the loaded
// registers at the latch, which waits for every outstanding load: one memory round trip a row.) Lanes past the
// range's end load its last chunk and weigh it 0 (their x digits and their all-ones pattern are zero); rows past the
// block's end load its last row again and store nothing. Ranges of one row combine with 64-bit atomics (exact in any
// order).
// K ranges of 4 KiB (4 chunks a lane), 2 KiB for rows of 8 KiB and more (7B down, 18944: 19.7 -> 18.6 us a call)
#ifndef ROWMAJ_LONG_K
#define ROWMAJ_LONG_K 8192
#endif
#ifndef ROWMAJ_WAVES
#define ROWMAJ_WAVES 2048                 // waves to aim for: rows per wave = N x ranges / ROWMAJ_WAVES (1..8)
#endif

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

#ifndef ROWMAJ_DPP
#define ROWMAJ_DPP 1
#endif
#ifndef ROWMAJ_BR
#define ROWMAJ_BR 1
#endif

template <int CH>
struct RowMajRow {
  v4i w[CH];
  int64_t m[CH];
};

template <bool NT, int CH>
__device__ __forceinline__ void rowmaj_load(RowMajRow<CH>& R_, const int8_t* __restrict__ wT, const int64_t* __restrict__ Mg,
                                            int n, int K, int G, int kb0, int nck, int lane) {
  const int8_t* wr = wT + (size_t)n * K + kb0;
  const int64_t* mr = Mg + (size_t)n * G + kb0 / 128;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ci = lane + 64 * c < nck ? lane + 64 * c : nck - 1;   // chunk index inside the range
    const v4i* p = reinterpret_cast<const v4i*>(wr + 16 * ci);
    R_.w[c] = NT ? __builtin_nontemporal_load(p) : *p;
    R_.m[c] = mr[ci >> 3];
  }
}

// BR: one block per row block with one wave per K range (blockDim = 64 nranges, at most ROWMAJ_BR_MAX): the ranges'
// row totals are added in LDS and stored once (no atomics, no clearing launch before)
#define ROWMAJ_BR_MAX 16
template <bool NT, int CH, int RPW, bool BR = false>
__global__ __launch_bounds__(BR ? 64 * ROWMAJ_BR_MAX : 256) void k_gemv_rowmajor(
    const int16_t* __restrict__ x, const int8_t* __restrict__ wT, const int64_t* __restrict__ Mg, int64_t* __restrict__ out,
    int N, int K, int G, int nranges, int out_mode) {
  constexpr int rpw = RPW;
  __shared__ int64_t red[BR ? ROWMAJ_BR_MAX : 1][RPW];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(BR ? (int)blockIdx.x * nranges + (int)(threadIdx.x >> 6)
                                                    : (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));   // rows and range: scalar
  const int nrb = (N + rpw - 1) / rpw;
  if (!BR && wid >= nrb * nranges) return;
  const int rb = wid / nranges, kr = wid - rb * nranges;
  const int kb0 = kr * CH * 1024;
  const int nck = ((K - kb0 < CH * 1024 ? K - kb0 : CH * 1024)) / 16;   // 16-byte chunks in the range
  const int n0 = rb * rpw, n1 = n0 + rpw < N ? n0 + rpw : N;
  // the lane's x digits, one 16-byte chunk of k per slot, and its all-ones pattern (zero past the range)
  v4i xh[CH], xl[CH];
  int ones[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const v4i zero = {0, 0, 0, 0};
    ones[c] = lane + 64 * c < nck ? 0x01010101 : 0;
    if (lane + 64 * c < nck) {
      const v4i* xp = reinterpret_cast<const v4i*>(x + kb0 + 16 * (lane + 64 * c));
      split_a16(xp[0], xp[1], xh[c], xl[c]);
    } else {
      xh[c] = zero;
      xl[c] = zero;
    }
  }
  auto row = [&](int r) { return n0 + r < n1 ? n0 + r : n1 - 1; };   // past the block's end: its last row again
  RowMajRow<CH> rr[2];
  rowmaj_load<NT, CH>(rr[0], wT, Mg, row(0), K, G, kb0, nck, lane);
  if (RPW > 1) rowmaj_load<NT, CH>(rr[1], wT, Mg, row(1), K, G, kb0, nck, lane);
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    RowMajRow<CH>& cur = rr[r & 1];
    int64_t part = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int sh = 0, sl = 0, s1 = 0;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        sh = dot4(cur.w[c][d], xh[c][d], sh);
        sl = dot4(cur.w[c][d], xl[c][d], sl);
        s1 = dot4(cur.w[c][d], ones[c], s1);
      }
      part += (int64_t)((sh << 8) + sl + (s1 << 7)) * cur.m[c];   // a = 0 past the range
    }
    if (r + 2 < RPW) rowmaj_load<NT, CH>(cur, wT, Mg, row(r + 2), K, G, kb0, nck, lane);
    if (ROWMAJ_DPP) {
      part = wave_sum64(part);   // row-level data movement and four reads of lanes, not six LDS-crossbar exchanges
    } else {
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) part += __shfl_xor(part, o, 64);
    }
    if constexpr (BR) {
      if (lane == 0) red[kr][r] = part;
    } else if (lane == 0 && n0 + r < n1) {
      if (out_mode)
        atomicAdd(reinterpret_cast<unsigned long long*>(out + n0 + r), (unsigned long long)part);
      else
        out[n0 + r] = part;
    }
  }
  if constexpr (BR) {
    __syncthreads();
    if (kr == 0 && lane < RPW && n0 + lane < n1) {
      uint64_t tot = 0;
      for (int k = 0; k < nranges; ++k) tot += (uint64_t)red[k][lane];
      out[n0 + lane] = (int64_t)tot;
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

// Work split: about GEMV_WAVES waves over the chip, groups spread evenly over the splits of a row block.
#ifndef GEMV_WAVES
#define GEMV_WAVES 3072
#endif
// ... and for int16 decode rows (R <= 4): 7B bs1 decode 2.104-2.122 -> 2.090-2.104 ms a step, 14B 4.174-4.183 ->
// 4.150-4.156 against 3072 (the down GEMV's 148 groups in 74 splits instead of 55); 6144 and 8192 slower, bs8 and 0.5B
// unchanged. int8 rows keep 3072: their large GEMVs then fit one round of 16-wave blocks (down: 56 x 55 tasks)
#ifndef GEMV_DECODE_WAVES
#define GEMV_DECODE_WAVES 4096
#endif
#ifndef GEMV_NT
#define GEMV_NT 1
#endif
// prefill rows up to this many GEMV row chunks run as chunked GEMVs rather than as the GEMM
// compute units of one MI355X (8 XCDs x 32): the fallback when the device cannot be queried
#ifndef GEMV_CUS
#define GEMV_CUS 256
#endif
// compute units of the current device (cached per device)
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return GEMV_CUS;
  if (cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = GEMV_CUS;
    cus[dev] = n;
  }
  return cus[dev];
}
#ifndef GEMV_CHUNKS_MAX
#define GEMV_CHUNKS_MAX 1
#endif
#define WIDE_A16_CHUNKS_MAX 3
// Above 4 rows each wave adds 64 x 16 int64 partial totals with atomics, so fewer group splits pay for most shapes.
// Measured at 8 and 16 rows on the 7B shapes (us, int16 / int8 rows at 16): q|k|v 19.2 -> 11.3 / 17.9 -> 10.1 and
// o 15.3 -> 11.3 / 13.7 -> 9.7 at 768 waves instead of 3072; gate|up (592 row blocks) 39.9 -> 32.6 at 1536 for int16
// rows; int8 gate|up and down (148 groups) stay fastest at 3072.
static int64_t gemv_waves(int64_t nbs, int G, int R, int abits) {
  if (R <= 4) return abits == 15 ? GEMV_DECODE_WAVES : GEMV_WAVES;
  if (abits == 15) return nbs > 256 ? 1536 : 768;
  return (nbs > 256 || G > 64) ? GEMV_WAVES : 768;
}
static int gemv_nsplit(int N, int G, int R = 1, int abits = 15) {
  const int64_t nbs = (N + 63) / 64;
  const int64_t waves = gemv_waves(nbs, G, R, abits);
  int64_t ns = (waves + nbs - 1) / nbs;
  if (ns < 1) ns = 1;
  if (ns > G) ns = G;
  return (int)ns;
}

// accumulate: t += x.W (t holds the caller's running total, e.g. zeros left by a consumer kernel);
// otherwise t is overwritten (zero-filled first when the row blocks are split).
int gemm_mfma(const void* x, int abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int M, int N,
              int K, hipStream_t st, bool zeroed);

// colterm (int16 rows only): the colsum term comes from colterm instead of an all-ones row, so R <= 16
int gemv_launch(const void* x, int abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int R, int N,
                int K, hipStream_t st, bool accumulate, const int64_t* colterm = nullptr) {
  const int G = K / 128;
  const int nsplit = gemv_nsplit(N, G, R, abits);
  const int out_mode = (accumulate || nsplit > 1) ? 1 : 0;
  if (!accumulate && nsplit > 1) {
    int e = zero_bytes(t, (int64_t)R * N * 8, st);
    if (e) return e;
  }
  const int tasks = ((N + 63) / 64) * nsplit;
  // Large int8-activation weights whose tasks fit the CUs in one round of 16-wave blocks run with 1024
  // threads per block: 16 consecutive tasks (neighbouring weight blocks) on one CU. Measured at R = 1:
  // 37888x3584 24.3 -> 22.8 us, 3584x18944 13.7 -> 13.3 us; smaller weights and the 152064-row head
  // (two rounds) run faster with 256-thread blocks, and int16 activations need more than the 128 VGPRs
  // a 1024-thread block leaves each wave.
  const bool wide = abits == 7 && (int64_t)N * K >= (32LL << 20) && (tasks + 15) / 16 <= device_cus();
  const int bw = wide ? 16 : 4;
  dim3 grid((tasks + bw - 1) / bw), block(64 * bw);
#define GEMV_GO(AB, VR, BW)                                                                                          \
  do {                                                                                                               \
    if (mh)                                                                                                          \
      hipLaunchKernelGGL((k_gemv_g128<AB, GEMV_NT != 0, VR, BW, false, true>), grid, block, 0, st, x, wp, mp, mh, t, R, N, \
                         K, G, nsplit, out_mode, nullptr);                                                          \
    else                                                                                                             \
      hipLaunchKernelGGL((k_gemv_g128<AB, GEMV_NT != 0, VR, BW>), grid, block, 0, st, x, wp, mp, mh, t, R, N, K, G,       \
                         nsplit, out_mode, nullptr);                                                                 \
  } while (0)
  const int vr = R <= 1 ? 1 : (R <= 2 ? 2 : 4);
  if (abits == 15 && colterm) {
#define GEMV_CT_GO(VR)                                                                                                 \
  do {                                                                                                                 \
    if (mh)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_g128<15, GEMV_NT != 0, VR, 4, true, true>), grid, block, 0, st, x, wp, mp, mh, t, R, N, K, \
                         G, nsplit, out_mode, colterm);                                                                \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_g128<15, GEMV_NT != 0, VR, 4, true>), grid, block, 0, st, x, wp, mp, mh, t, R, N, K, G,    \
                         nsplit, out_mode, colterm);                                                                   \
  } while (0)
    if (vr == 1) GEMV_CT_GO(1); else if (vr == 2) GEMV_CT_GO(2); else GEMV_CT_GO(4);
#undef GEMV_CT_GO
  } else if (abits == 15) {
    if (vr == 1) GEMV_GO(15, 1, 4); else if (vr == 2) GEMV_GO(15, 2, 4); else GEMV_GO(15, 4, 4);
  } else if (wide) {
    if (vr == 1) GEMV_GO(7, 1, 16); else if (vr == 2) GEMV_GO(7, 2, 16); else GEMV_GO(7, 4, 16);
  } else {
    if (vr == 1) GEMV_GO(7, 1, 4); else if (vr == 2) GEMV_GO(7, 2, 4); else GEMV_GO(7, 4, 4);
  }
#undef GEMV_GO
  return launch_status("gemv_g128");
}

// MoE decode: the routed experts' SwiGLU GEMV and the shared expert's (R rows of the same activations) in one launch:
// blocks below B1 are k_gemv_experts_swiglu's, the others k_gemv_gu_swiglu's (both 4 waves a block)
template <bool NT, int VR, bool WIDE>
__global__ __launch_bounds__(256) void k_moe_swiglu_pair(const int16_t* __restrict__ x, const int32_t* __restrict__ row_map,
                                                         const int8_t* __restrict__ ewp, const int16_t* __restrict__ emp,
                                                         int64_t w_stride, int64_t m_stride,
                                                         const int32_t* __restrict__ chunk_e,
                                                         const int32_t* __restrict__ chunk_p0,
                                                         const int32_t* __restrict__ chunk_n,
                                                         const int32_t* __restrict__ nchunks,
                                                         const int32_t* __restrict__ s_pair, const int32_t* __restrict__ silu,
                                                         int64_t* __restrict__ eh, int32_t* __restrict__ epart, int EI,
                                                         const int8_t* __restrict__ swp, const int16_t* __restrict__ smp,
                                                         const int16_t* __restrict__ smh, const int32_t* __restrict__ s,
                                                         int64_t* __restrict__ sh, int32_t* __restrict__ spart, int R, int SI,
                                                         int K, int B1, int B2) {
  if ((int)blockIdx.x < B1)
    experts_swiglu_body<NT, 4>(x, row_map, ewp, emp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, s_pair, silu,
                               eh, epart, EI, K, K / 128, blockIdx.x);
  else
    gu_swiglu_body<NT, VR, 1, 4, WIDE, 0>(x, swp, smp, smh, s, silu, sh, spart, nullptr, R, SI, K, K / 128, nullptr, nullptr,
                                           nullptr, nullptr, nullptr, nullptr, (int)blockIdx.x - B1, B2);
}

// ... and the two down GEMVs that quantise those SwiGLU rows: blocks below B1 are k_gemv_experts_xq's, the others
// k_gemv_g128_xq's; every block also clears its share of zero
template <bool NT, int VR, bool WIDE, int PLE, int PLS>
__global__ __launch_bounds__(256) void k_moe_qrow_pair(const int64_t* __restrict__ exs, int64_t eldx,
                                                       const int32_t* __restrict__ epart, int enparts,
                                                       const int8_t* __restrict__ ewp, const int16_t* __restrict__ emp,
                                                       int64_t w_stride, int64_t m_stride, const int32_t* __restrict__ chunk_e,
                                                       const int32_t* __restrict__ chunk_p0,
                                                       const int32_t* __restrict__ chunk_n,
                                                       const int32_t* __restrict__ nchunks, int64_t* __restrict__ et,
                                                       int32_t* __restrict__ es_out, int EN, int EK, int ensplit, int egmax,
                                                       const int64_t* __restrict__ sxs, int64_t sldx,
                                                       const int32_t* __restrict__ spart, int snparts,
                                                       const int8_t* __restrict__ swp, const int16_t* __restrict__ smp,
                                                       const int16_t* __restrict__ smh, int64_t* __restrict__ st,
                                                       int32_t* __restrict__ ss_out, int R, int SN, int SK, int snsplit,
                                                       int sgmax, int64_t* __restrict__ zero, int64_t zero_n, int B1) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < zero_n; i += (int64_t)gridDim.x * blockDim.x)
    zero[i] = 0;
  if ((int)blockIdx.x < B1)
    experts_xq_body<NT, PLE>(exs, eldx, epart, enparts, ewp, emp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, et,
                             es_out, EN, EK, EK / 128, ensplit, egmax, blockIdx.x);
  else
    g128_xq_body<15, NT, VR, WIDE, PLS>(sxs, sldx, spart, snparts, swp, smp, smh, st, ss_out, R, SN, SK, SK / 128, snsplit,
                                        sgmax, (int)blockIdx.x - B1);
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

extern "C" int exact_gemv_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                               int64_t* t, int32_t R, int32_t N, int32_t K, void* stream) {
  int e = check_linear(x, abits, wp, mp, t, R, N, K);
  if (e) return e;
  const int rmax = abits == 15 ? 15 : 16;   // one A row is the all-ones colsum row in the A16 mode
  if (R > rmax) return EXACT_E_UNSUPPORTED;
  return gemv_launch(x, abits, wp, mp, mh, t, R, N, K, as_stream(stream), false);
}

extern "C" int exact_gemv_g128_acc(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                   int64_t* t, int32_t R, int32_t N, int32_t K, void* stream) {
  int e = check_linear(x, abits, wp, mp, t, R, N, K);
  if (e) return e;
  if (R > (abits == 15 ? 15 : 16)) return EXACT_E_UNSUPPORTED;
  return gemv_launch(x, abits, wp, mp, mh, t, R, N, K, as_stream(stream), true);
}

extern "C" int exact_gemv(const int16_t* x, const int8_t* wT, const int64_t* Mg, int64_t* out, int32_t N, int32_t K,
                          void* stream) {
  if (!x || !wT || !Mg || !out || N <= 0 || K <= 0) return EXACT_E_ARG;
  if (K % 128) return EXACT_E_UNSUPPORTED;   // the reference reads Mg[n][k >> 7] and so assumes whole groups
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(wT) & 15) ||
      (reinterpret_cast<uintptr_t>(Mg) & 7) || (reinterpret_cast<uintptr_t>(out) & 7))
    return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int ch = K >= ROWMAJ_LONG_K ? 2 : 4;
  const int nranges = (K + ch * 1024 - 1) / (ch * 1024);
  const int64_t rq = (int64_t)N * nranges / ROWMAJ_WAVES;
  const int rpw = rq >= 8 ? 8 : (rq >= 4 ? 4 : (rq >= 2 ? 2 : 1));   // rows per wave: a power of two up to 8
  const int64_t waves = (((int64_t)N + rpw - 1) / rpw) * nranges;
  if (waves > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  hipStream_t st = as_stream(stream);
  // several K ranges: one block per row block, its waves the ranges (ROWMAJ_BR), else atomics into a cleared output
  const bool br = ROWMAJ_BR && nranges > 1 && nranges <= ROWMAJ_BR_MAX;
  if (nranges > 1 && !br) {
    int e = zero_bytes(out, (int64_t)N * 8, st);
    if (e) return e;
  }
  const dim3 grid((unsigned)(br ? (N + rpw - 1) / rpw : (waves + 3) / 4)), block(br ? 64 * nranges : 256);
  const int mode = nranges > 1 ? 1 : 0;
#define ROWMAJ_GO(C, P)                                                                                                \
  do {                                                                                                                 \
    if (br)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_rowmajor<GEMV_NT != 0, C, P, true>), grid, block, 0, st, x, wT, Mg, out, N, K, G, nranges, \
                         mode);                                                                                        \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_rowmajor<GEMV_NT != 0, C, P>), grid, block, 0, st, x, wT, Mg, out, N, K, G, nranges, mode); \
  } while (0)
  if (ch == 2) {
    if (rpw == 8) ROWMAJ_GO(2, 8); else if (rpw == 4) ROWMAJ_GO(2, 4); else if (rpw == 2) ROWMAJ_GO(2, 2); else ROWMAJ_GO(2, 1);
  } else {
    if (rpw == 8) ROWMAJ_GO(4, 8); else if (rpw == 4) ROWMAJ_GO(4, 4); else if (rpw == 2) ROWMAJ_GO(4, 2); else ROWMAJ_GO(4, 1);
  }
#undef ROWMAJ_GO
  return launch_status("gemv");
}

// rows of one norm-fused GEMV launch (each block runs the row program once per row) and the row width its 256 threads
// hold in registers (24 values each)
#define GEMV_NORM_ROWS 2
#ifndef GEMV_NORM_BW8_K
#define GEMV_NORM_BW8_K 1024   // rows wider than this (MoE q|k|v 6144 x 2048, A/B: 1.98-2.00 -> 1.95-1.97 ms a step)
#endif
#define GEMV_NORM_KMAX (256 * 24)
#ifndef GEMV_NORM_EPT10
#define GEMV_NORM_EPT10 1
#endif

// rows wider than GEMV_NORM_BW8_K whose group-split tasks do not fit one round of 8-wave blocks: the split capped so
// that they do, when that leaves at least GEMV_NORM_FIT_MIN splits (0: never)
#ifndef GEMV_NORM_FIT_MIN
#define GEMV_NORM_FIT_MIN 8
#endif

// group split and waves per block of exact_gemv_g128_norm_acc on `cus` compute units: 8-wave blocks, one per CU (each
// CU then normalises the row once), for rows wider than GEMV_NORM_BW8_K whose tasks fit one round or are capped to;
// else 4-wave blocks, every block normalising the row
static int norm_split(int R, int N, int K, int cus, int* bw) {
  const int64_t nbs = (N + 63) / 64;
  const int ns = gemv_nsplit(N, K / 128, R, 15);
  *bw = 4;
  if (K <= GEMV_NORM_BW8_K) return ns;
  if ((nbs * ns + 7) / 8 <= cus) {
    *bw = 8;
    return ns;
  }
  const int64_t cap = (int64_t)cus * 8 / nbs;
  if (GEMV_NORM_FIT_MIN > 0 && cap >= GEMV_NORM_FIT_MIN) {
    *bw = 8;
    return (int)cap;
  }
  return ns;
}
static int norm_block_waves(int R, int N, int K, int cus) {
  int bw;
  (void)norm_split(R, N, K, cus, &bw);
  return bw;
}

extern "C" int exact_gemv_g128_norm_acc_blockwaves(int32_t R, int32_t N, int32_t K, int32_t cus) {
  if (R <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
  return norm_block_waves(R, N, K, cus > 0 ? cus : device_cus());
}

extern "C" int exact_gemv_g128_norm_acc(const int64_t* x_in, int64_t* x_out, const int64_t* res_t, const int32_t* res_s,
                                        const int64_t* g, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                        int64_t* t, int32_t* s_out, int16_t* xq_out, int32_t R, int32_t N, int32_t K,
                                        void* stream) {
  if (!x_in || !g || !wp || !mp || !t || R <= 0 || N <= 0 || K <= 0 || (res_t && !res_s)) return EXACT_E_ARG;
  if (x_out && (x_out == x_in || x_out == res_t)) return EXACT_E_ARG;   // the other blocks still read x_in / res_t
  if (K % 128 || K > GEMV_NORM_KMAX || R > GEMV_NORM_ROWS) return EXACT_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(wp) & 15) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  int bw;
  const int nsplit = norm_split(R, N, K, device_cus(), &bw);   // 8-wave blocks: see the kernel
  const bool bw8 = bw == 8;
  const int64_t tasks = (int64_t)((N + 63) / 64) * nsplit;
  const size_t lds = (size_t)R * K * 2;
  hipStream_t st = as_stream(stream);
  dim3 grid((unsigned)((tasks + bw - 1) / bw)), block(64 * bw);
  const int ept = (K + 64 * bw - 1) / (64 * bw);
#define NORM_GO_BW(VR, E, BW)                                                                                           \
  do {                                                                                                                  \
    if (mh)                                                                                                             \
      hipLaunchKernelGGL((k_gemv_g128_norm<GEMV_NT != 0, VR, E, true, BW>), grid, block, lds, st, x_in, x_out, res_t, res_s,\
                         g, wp, mp, mh, t, s_out, xq_out, R, N, K, G, nsplit);                                          \
    else                                                                                                                \
      hipLaunchKernelGGL((k_gemv_g128_norm<GEMV_NT != 0, VR, E, false, BW>), grid, block, lds, st, x_in, x_out, res_t,     \
                         res_s, g, wp, mp, mh, t, s_out, xq_out, R, N, K, G, nsplit);                                   \
  } while (0)
#define NORM_GO(VR, E)                                                                                                  \
  do {                                                                                                                  \
    if (bw8) NORM_GO_BW(VR, E, 8); else NORM_GO_BW(VR, E, 4);                                                           \
  } while (0)
#define NORM_EPT(VR)                                                                                                    \
  do {                                                                                                                  \
    if (ept <= 4) NORM_GO(VR, 4);                                                                                       \
    else if (ept == 7 && bw8) NORM_GO_BW(VR, 7, 8);   /* 3584-wide rows over 512 threads: no padded slots */            \
    else if (ept == 10 && bw8 && GEMV_NORM_EPT10) NORM_GO_BW(VR, 10, 8);   /* 5120-wide rows likewise */                   \
    else if (ept <= 8) NORM_GO(VR, 8);                                                                                  \
    else if (ept <= 14) NORM_GO(VR, 14);                                                                                \
    else if (ept <= 20) NORM_GO(VR, 20);                                                                                \
    else NORM_GO(VR, 24);                                                                                               \
  } while (0)
  if (R == 1) NORM_EPT(1); else NORM_EPT(2);
#undef NORM_EPT
#undef NORM_GO
#undef NORM_GO_BW
  return launch_status("gemv_g128_norm_acc");
}

// LDS of the quantised slices: 4 waves x R rows x gmax groups x 128 values
#define GEMV_XQ_LDS_MAX (64 * 1024)
// slice bit lengths per row beyond 64 (the SwiGLU GEMV writes one per 32 or 64 columns): up to 64 * XQ_PARTS_WIDE
#define XQ_PARTS_WIDE 16

extern "C" int exact_gemv_g128_qrow_acc(const int64_t* xs, int64_t ldx, const int32_t* part, int32_t nparts, int32_t abits,
                                        const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int32_t* s_out,
                                        int32_t R, int32_t N, int32_t K, int64_t* zero, int64_t zero_n, void* stream) {
  if (!xs || !part || !wp || !mp || !t || !s_out || R <= 0 || N <= 0 || K <= 0 || nparts <= 0 || ldx < K)
    return EXACT_E_ARG;
  if (zero_n < 0 || (zero_n > 0 && !zero)) return EXACT_E_ARG;
  if ((abits != 15 && abits != 7) || K % 128 || (reinterpret_cast<uintptr_t>(wp) & 15)) return EXACT_E_UNSUPPORTED;
  if (R > (abits == 15 ? 15 : 16)) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int nsplit = gemv_nsplit(N, G);
  const int gmax = (G + nsplit - 1) / nsplit;
  const size_t lds = (size_t)4 * R * gmax * 128 * (abits == 15 ? 2 : 1);
  if (lds > GEMV_XQ_LDS_MAX || gmax * 128 > 64 * XQ_LOADS || nparts > 64 * XQ_PARTS_WIDE) return EXACT_E_UNSUPPORTED;
  const int tasks = ((N + 63) / 64) * nsplit;
  dim3 grid((tasks + 3) / 4), block(256);
  hipStream_t st = as_stream(stream);
#define XQ_GO_PL(AB, VR, PL)                                                                                           \
  do {                                                                                                                 \
    if (mh)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_g128_xq<AB, GEMV_NT != 0, VR, true, PL>), grid, block, lds, st, xs, ldx, part, nparts, wp, \
                         mp, mh, t, s_out, R, N, K, G, nsplit, gmax, zero, zero_n);                                    \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_g128_xq<AB, GEMV_NT != 0, VR, false, PL>), grid, block, lds, st, xs, ldx, part, nparts,   \
                         wp, mp, mh, t, s_out, R, N, K, G, nsplit, gmax, zero, zero_n);                                \
  } while (0)
#define XQ_GO(AB, VR)                                                                                                  \
  do {                                                                                                                 \
    if (nparts <= 64) XQ_GO_PL(AB, VR, 1);                                                                             \
    else if (nparts <= 256) XQ_GO_PL(AB, VR, 4);                                                                       \
    else XQ_GO_PL(AB, VR, XQ_PARTS_WIDE);                                                                              \
  } while (0)
  const int vr = R <= 1 ? 1 : (R <= 2 ? 2 : 4);
  if (abits == 15) {
    if (vr == 1) XQ_GO(15, 1); else if (vr == 2) XQ_GO(15, 2); else XQ_GO(15, 4);
  } else {
    if (vr == 1) XQ_GO(7, 1); else if (vr == 2) XQ_GO(7, 2); else XQ_GO(7, 4);
  }
#undef XQ_GO
#undef XQ_GO_PL
  return launch_status("gemv_g128_qrow_acc");
}

// The SwiGLU GEMV's blocks: GEMV_GU_NPB pairs of 32 gate columns x GEMV_GU_KS k parts (rows above 2), GEMV_GU_KS1
// k parts for one or two rows (the MoE shared expert's 11264 x 2048 at bs1: 4 parts of 4 groups, 1.725-1.740 ->
// 1.704-1.723 ms a step; at 8 rows 4 parts cost the 14B 1%)
#ifndef GEMV_GU_KS
#define GEMV_GU_KS 2
#endif
#ifndef GEMV_GU_KS1
#define GEMV_GU_KS1 4
#endif
#ifndef GEMV_GU_NPB
#define GEMV_GU_NPB 1
#endif

extern "C" int exact_gemv_g128_swiglu(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                      const int32_t* s, const int32_t* silu, int64_t* h, int32_t* part, int64_t* t,
                                      int32_t R, int32_t I, int32_t K, void* stream) {
  if (!x || !wp || !mp || !s || !silu || !h || !part || R <= 0 || I <= 0 || K <= 0) return EXACT_E_ARG;
  if (R > 8 || I % 64 || K % 128) return EXACT_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(wp) & 15)) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int ks = R <= 2 ? GEMV_GU_KS1 : GEMV_GU_KS;
  dim3 grid((unsigned)(I / (32 * GEMV_GU_NPB))), block(64 * GEMV_GU_NPB * ks);
  hipStream_t st = as_stream(stream);
#define GU_GO(VR, KS)                                                                                                  \
  do {                                                                                                                 \
    if (mh)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, GEMV_GU_NPB, KS, true>), grid, block, 0, st, x, wp, mp, mh, s,  \
                         silu, h, part, t, R, I, K, G);                                                                \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, GEMV_GU_NPB, KS, false>), grid, block, 0, st, x, wp, mp, mh, s, \
                         silu, h, part, t, R, I, K, G);                                                                \
  } while (0)
  if (R == 1) GU_GO(1, GEMV_GU_KS1); else if (R == 2) GU_GO(2, GEMV_GU_KS1); else GU_GO(4, GEMV_GU_KS);
#undef GU_GO
  return launch_status("gemv_g128_swiglu");
}

// rows of one norm-fused SwiGLU GEMV launch, its blocks (NPB pairs as exact_gemv_g128_swiglu, so part has the same
// slices, x KS k parts) and the row width their threads hold (16 values each)
#define GEMV_NSW_ROWS 2
#define GEMV_NSW_NPB GEMV_GU_NPB
#ifndef GEMV_NSW_KS
#define GEMV_NSW_KS 8   // 0.5B bs1 decode (2 values a thread of its 896-wide rows), A/B: KS 2 0.768-0.779 ms a step,
                        // 4 0.744-0.753, 7 0.737-0.747, 8 0.736-0.745
#endif
#define GEMV_NSW_THREADS (64 * GEMV_NSW_NPB * GEMV_NSW_KS)
#define GEMV_NSW_KMAX (128 * 16)
#define GEMV_NSW_WIDE_KMAX (128 * 64)   // wider rows (up to this): 8-wave blocks, see the launcher
// rows of up to 4 values a thread (the 0.5B's 896 over 256 threads) hold 4, not 8 with padded slots: 0.5B bs1
// decode 0.771-0.773 -> 0.749-0.750 ms a step
#ifndef GEMV_NSW_EPT4
#define GEMV_NSW_EPT4 1
#endif

extern "C" int exact_gemv_g128_norm_swiglu(const int64_t* x_in, int64_t* x_out, const int64_t* res_t, const int32_t* res_s,
                                           const int64_t* g, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                           int32_t* s_out, const int32_t* silu, int64_t* h, int32_t* part, int64_t* t,
                                           int32_t R, int32_t I, int32_t K, void* stream) {
  if (!x_in || !g || !wp || !mp || !s_out || !silu || !h || !part || R <= 0 || I <= 0 || K <= 0 || (res_t && !res_s))
    return EXACT_E_ARG;
  if (x_out && (x_out == x_in || x_out == res_t)) return EXACT_E_ARG;   // the other blocks still read x_in / res_t
  if (R > GEMV_NSW_ROWS || I % 64 || K % 128 || K > GEMV_NSW_WIDE_KMAX) return EXACT_E_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(wp) & 15) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  if (K > GEMV_NSW_KMAX) {
    // wide rows: 8-wave blocks, each normalising the rows once, as many as the CUs take in one round: pairs of 32 gate
    // columns x k parts 2 x 4 when I / 64 blocks fit (14B, I = 13824: 216 blocks; A/B 4.15 -> 3.91 ms a decode step),
    // else 4 x 2 (7B, I = 18944: 148 blocks; 2.10 -> 1.99 ms; as 2 x 4, 296 blocks: 2.27)
    if (I % 128 && I / 64 > device_cus()) return EXACT_E_UNSUPPORTED;
    const bool np2 = I / 64 <= device_cus();
    dim3 gridw((unsigned)(I / (np2 ? 64 : 128))), blockw(512);
    const size_t ldsw = (size_t)R * K * 2;
    hipStream_t stw = as_stream(stream);
    const int eptw = (K + 511) / 512;
#define NSWW_GO2(VR, E, NPBW, KSW)                                                                                     \
  do {                                                                                                                 \
    if (mh)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, NPBW, KSW, true, E>), gridw, blockw, ldsw, stw, nullptr, wp,  \
                         mp, mh, nullptr, silu, h, part, t, R, I, K, G, x_in, x_out, res_t, res_s, g, s_out);           \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, NPBW, KSW, false, E>), gridw, blockw, ldsw, stw, nullptr, wp, \
                         mp, mh, nullptr, silu, h, part, t, R, I, K, G, x_in, x_out, res_t, res_s, g, s_out);           \
  } while (0)
#define NSWW_GO(VR, E)                                                                                                 \
  do {                                                                                                                 \
    if (np2) NSWW_GO2(VR, E, 2, 4); else NSWW_GO2(VR, E, 4, 2);                                                        \
  } while (0)
#define NSWW_EPT(VR)                                                                                                   \
  do {                                                                                                                 \
    if (eptw <= 7) NSWW_GO(VR, 7);                                                                                     \
    else if (eptw <= 10) NSWW_GO(VR, 10);                                                                              \
    else NSWW_GO(VR, 16);                                                                                              \
  } while (0)
    if (R == 1) NSWW_EPT(1); else NSWW_EPT(2);
#undef NSWW_EPT
#undef NSWW_GO
#undef NSWW_GO2
    return launch_status("gemv_g128_norm_swiglu");
  }
  if (I % (32 * GEMV_NSW_NPB)) return EXACT_E_UNSUPPORTED;
  dim3 grid((unsigned)(I / (32 * GEMV_NSW_NPB))), block(GEMV_NSW_THREADS);
  const size_t lds = (size_t)R * K * 2;
  hipStream_t st = as_stream(stream);
  const int ept = (K + GEMV_NSW_THREADS - 1) / GEMV_NSW_THREADS;
#define NSW_GO(VR, E)                                                                                                  \
  do {                                                                                                                 \
    if (mh)                                                                                                            \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, GEMV_NSW_NPB, GEMV_NSW_KS, true, E>), grid, block, lds, st,     \
                         nullptr, wp, mp, mh, nullptr, silu, h, part, t, R, I, K, G, x_in, x_out, res_t, res_s, g, s_out);   \
    else                                                                                                               \
      hipLaunchKernelGGL((k_gemv_gu_swiglu<GEMV_NT != 0, VR, GEMV_NSW_NPB, GEMV_NSW_KS, false, E>), grid, block, lds, st,    \
                         nullptr, wp, mp, mh, nullptr, silu, h, part, t, R, I, K, G, x_in, x_out, res_t, res_s, g, s_out);   \
  } while (0)
  if (R == 1) {
    if (ept <= 2) NSW_GO(1, 2); else if (ept <= 4 && GEMV_NSW_EPT4) NSW_GO(1, 4); else if (ept <= 8) NSW_GO(1, 8); else NSW_GO(1, 16);
  } else {
    if (ept <= 2) NSW_GO(2, 2); else if (ept <= 4 && GEMV_NSW_EPT4) NSW_GO(2, 4); else if (ept <= 8) NSW_GO(2, 8); else NSW_GO(2, 16);
  }
#undef NSW_GO
  return launch_status("gemv_g128_norm_swiglu");
}

static int gemm_entry(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t,
                      int32_t R, int32_t N, int32_t K, void* stream, bool zeroed) {
  int e = check_linear(x, abits, wp, mp, t, R, N, K);
  if (e) return e;
  const int rmax = abits == 15 ? 15 : 16;
  // int16 rows with wide scales have no MFMA kernel behind this entry (the digit-row entry exact_gemm_g128_a16 is
  // theirs): they keep the GEMV row chunks up to WIDE_A16_CHUNKS_MAX x 15 rows, and above that gemm_mfma refuses them
  const int chunks_max = (abits == 15 && mh) ? WIDE_A16_CHUNKS_MAX : GEMV_CHUNKS_MAX;
  if (R > chunks_max * rmax) return gemm_mfma(x, abits, wp, mp, mh, t, R, N, K, as_stream(stream), zeroed);
  // Up to GEMV_CHUNKS_MAX row chunks: one GEMV per chunk streams the weights once per chunk. One chunk beats the
  // GEMM's 128-row tiles (mostly padding at these R); a second weight pass does not (int8-row 7B prefill, ms: 32 tokens
  // as 2 chunks 5.79, on the GEMM 4.82; 48 tokens as 3 chunks 8.23, on the GEMM 5.11).
  const size_t xrow = (size_t)K * (abits == 15 ? 2 : 1);
  for (int r0 = 0; r0 < R; r0 += rmax) {
    const int rows = R - r0 < rmax ? R - r0 : rmax;
    e = gemv_launch(static_cast<const int8_t*>(x) + r0 * xrow, abits, wp, mp, mh, t + (size_t)r0 * N, rows, N, K,
                    as_stream(stream), zeroed);
    if (e) return e;
  }
  return EXACT_OK;
}

extern "C" int exact_gemm_g128(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                               int64_t* t, int32_t R, int32_t N, int32_t K, void* stream) {
  return gemm_entry(x, abits, wp, mp, mh, t, R, N, K, stream, false);
}

extern "C" int exact_gemm_g128_zeroed(const void* x, int32_t abits, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                      int64_t* t, int32_t R, int32_t N, int32_t K, void* stream) {
  return gemm_entry(x, abits, wp, mp, mh, t, R, N, K, stream, true);
}

extern "C" int exact_gemv_g128_experts(const void* x, int32_t abits, const int32_t* row_map, const int8_t* wp,
                                       const int16_t* mp, int64_t w_stride, int64_t m_stride, const int32_t* chunk_e,
                                       const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks,
                                       int32_t max_chunks, int64_t* t, int32_t N, int32_t K, void* stream) {
  int e = check_linear(x, abits, wp, mp, t, 1, N, K);
  if (e) return e;
  if (!chunk_e || !chunk_p0 || !chunk_n || !nchunks || max_chunks <= 0 || w_stride < 0 || m_stride < 0) return EXACT_E_ARG;
  if ((w_stride & 15) || (m_stride & 7)) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int64_t nbs = (N + 63) / 64;
  int64_t ns = (GEMV_WAVES + (int64_t)max_chunks * nbs - 1) / ((int64_t)max_chunks * nbs);
  ns = ns < 1 ? 1 : (ns > G ? G : ns);
  const int64_t tasks = (int64_t)max_chunks * nbs * ns;
  if (tasks > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  dim3 grid((unsigned)((tasks + 3) / 4)), block(256);
  if (abits == 15)
    hipLaunchKernelGGL((k_gemv_experts<15, GEMV_NT != 0>), grid, block, 0, as_stream(stream), x, row_map, wp, mp, w_stride,
                       m_stride, chunk_e, chunk_p0, chunk_n, nchunks, t, N, K, G, (int)ns);
  else
    hipLaunchKernelGGL((k_gemv_experts<7, GEMV_NT != 0>), grid, block, 0, as_stream(stream), x, row_map, wp, mp, w_stride,
                       m_stride, chunk_e, chunk_p0, chunk_n, nchunks, t, N, K, G, (int)ns);
  return launch_status("gemv_g128_experts");
}

// dispatched chunks of at most this many pairs take the fused expert GEMVs below
#define EXPERT_FUSE_CHUNK 4

static int check_chunks(const int32_t* chunk_e, const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks,
                        int32_t max_chunks, int32_t chunk, int64_t w_stride, int64_t m_stride) {
  if (!chunk_e || !chunk_p0 || !chunk_n || !nchunks || max_chunks <= 0 || w_stride < 0 || m_stride < 0 || chunk <= 0)
    return EXACT_E_ARG;
  if (chunk > EXPERT_FUSE_CHUNK || (w_stride & 15) || (m_stride & 7)) return EXACT_E_UNSUPPORTED;
  return EXACT_OK;
}

#ifndef GEMV_EXP_KS
#define GEMV_EXP_KS 4
#endif

extern "C" int exact_gemv_g128_experts_swiglu(const int16_t* x, const int32_t* row_map, const int8_t* wp, const int16_t* mp,
                                              int64_t w_stride, int64_t m_stride, const int32_t* chunk_e,
                                              const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks,
                                              int32_t max_chunks, int32_t chunk, const int32_t* s_pair,
                                              const int32_t* silu, int64_t* h, int32_t* part, int32_t I, int32_t K,
                                              void* stream) {
  if (!x || !wp || !mp || !s_pair || !silu || !h || !part || I <= 0 || K <= 0) return EXACT_E_ARG;
  int e = check_chunks(chunk_e, chunk_p0, chunk_n, nchunks, max_chunks, chunk, w_stride, m_stride);
  if (e) return e;
  if (I % 64 || K % 128 || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(wp) & 15))
    return EXACT_E_UNSUPPORTED;
  const int64_t blocks = (int64_t)max_chunks * (I / 32);
  if (blocks > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  hipLaunchKernelGGL((k_gemv_experts_swiglu<GEMV_NT != 0, GEMV_EXP_KS>), dim3((unsigned)blocks), dim3(64 * GEMV_EXP_KS), 0,
                     as_stream(stream), x, row_map, wp, mp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, s_pair,
                     silu, h, part, I, K, K / 128);
  return launch_status("gemv_g128_experts_swiglu");
}

extern "C" int exact_gemv_g128_experts_qrow_acc(const int64_t* xs, int64_t ldx, const int32_t* part, int32_t nparts,
                                                const int8_t* wp, const int16_t* mp, int64_t w_stride, int64_t m_stride,
                                                const int32_t* chunk_e, const int32_t* chunk_p0, const int32_t* chunk_n,
                                                const int32_t* nchunks, int32_t max_chunks, int32_t chunk, int64_t* t,
                                                int32_t* s_out, int32_t N, int32_t K, void* stream) {
  if (!xs || !part || !wp || !mp || !t || !s_out || N <= 0 || K <= 0 || nparts <= 0 || ldx < K) return EXACT_E_ARG;
  int e = check_chunks(chunk_e, chunk_p0, chunk_n, nchunks, max_chunks, chunk, w_stride, m_stride);
  if (e) return e;
  if (K % 128 || (reinterpret_cast<uintptr_t>(wp) & 15)) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int64_t nbs = (N + 63) / 64;
  int64_t ns = (GEMV_WAVES + (int64_t)max_chunks * nbs - 1) / ((int64_t)max_chunks * nbs);
  ns = ns < 1 ? 1 : (ns > G ? G : ns);
  const int gmax = (int)((G + ns - 1) / ns);
  const size_t lds = (size_t)4 * EXPERT_FUSE_CHUNK * gmax * 128 * 2;
  if (lds > GEMV_XQ_LDS_MAX || gmax * 128 > 64 * XQ_LOADS || nparts > 64 * XQ_PARTS_WIDE) return EXACT_E_UNSUPPORTED;
  const int64_t tasks = (int64_t)max_chunks * nbs * ns;
  if (tasks > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  dim3 grid((unsigned)((tasks + 3) / 4)), block(256);
  hipStream_t st = as_stream(stream);
  if (nparts <= 64)
    hipLaunchKernelGGL((k_gemv_experts_xq<GEMV_NT != 0, 1>), grid, block, lds, st, xs, ldx, part, nparts, wp, mp, w_stride,
                       m_stride, chunk_e, chunk_p0, chunk_n, nchunks, t, s_out, N, K, G, (int)ns, gmax);
  else
    hipLaunchKernelGGL((k_gemv_experts_xq<GEMV_NT != 0, XQ_PARTS_WIDE>), grid, block, lds, st, xs, ldx, part, nparts, wp, mp,
                       w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, t, s_out, N, K, G, (int)ns, gmax);
  return launch_status("gemv_g128_experts_qrow_acc");
}

extern "C" int exact_moe_swiglu_pair(const int16_t* x, const int32_t* row_map, const int8_t* ewp, const int16_t* emp,
                                     int64_t w_stride, int64_t m_stride, const int32_t* chunk_e, const int32_t* chunk_p0,
                                     const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks, int32_t chunk,
                                     const int32_t* s_pair, const int32_t* silu, int64_t* eh, int32_t* epart, int32_t EI,
                                     const int8_t* swp, const int16_t* smp, const int16_t* smh, const int32_t* s, int64_t* sh,
                                     int32_t* spart, int32_t R, int32_t SI, int32_t K, void* stream) {
  if (!x || !ewp || !emp || !s_pair || !silu || !eh || !epart || !swp || !smp || !s || !sh || !spart) return EXACT_E_ARG;
  if (EI <= 0 || SI <= 0 || K <= 0 || R <= 0) return EXACT_E_ARG;
  int e = check_chunks(chunk_e, chunk_p0, chunk_n, nchunks, max_chunks, chunk, w_stride, m_stride);
  if (e) return e;
  if (R > 2 || EI % 64 || SI % 64 || K % 128 || GEMV_EXP_KS != 4 || GEMV_GU_KS1 != 4 || GEMV_GU_NPB != 1)
    return EXACT_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(ewp) & 15) || (reinterpret_cast<uintptr_t>(swp) & 15))
    return EXACT_E_UNSUPPORTED;
  const int64_t B1 = (int64_t)max_chunks * (EI / 32), B2 = SI / 32;
  if (B1 + B2 > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  hipStream_t st = as_stream(stream);
#define PAIR_GO(VR, W)                                                                                                 \
  hipLaunchKernelGGL((k_moe_swiglu_pair<GEMV_NT != 0, VR, W>), dim3((unsigned)(B1 + B2)), dim3(256), 0, st, x, row_map, ewp, \
                     emp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, s_pair, silu, eh, epart, EI, swp, smp,  \
                     smh, s, sh, spart, R, SI, K, (int)B1, (int)B2)
  if (smh) {
    if (R == 1) PAIR_GO(1, true); else PAIR_GO(2, true);
  } else {
    if (R == 1) PAIR_GO(1, false); else PAIR_GO(2, false);
  }
#undef PAIR_GO
  return launch_status("moe_swiglu_pair");
}

extern "C" int exact_moe_qrow_pair(const int64_t* exs, int64_t eldx, const int32_t* epart, int32_t enparts, const int8_t* ewp,
                                   const int16_t* emp, int64_t w_stride, int64_t m_stride, const int32_t* chunk_e,
                                   const int32_t* chunk_p0, const int32_t* chunk_n, const int32_t* nchunks, int32_t max_chunks,
                                   int32_t chunk, int64_t* et, int32_t* es_out, int32_t EN, int32_t EK, const int64_t* sxs,
                                   int64_t sldx, const int32_t* spart, int32_t snparts, const int8_t* swp, const int16_t* smp,
                                   const int16_t* smh, int64_t* st, int32_t* ss_out, int32_t R, int32_t SN, int32_t SK,
                                   int64_t* zero, int64_t zero_n, void* stream) {
  if (!exs || !epart || !ewp || !emp || !et || !es_out || !sxs || !spart || !swp || !smp || !st || !ss_out) return EXACT_E_ARG;
  if (EN <= 0 || EK <= 0 || SN <= 0 || SK <= 0 || R <= 0 || enparts <= 0 || snparts <= 0 || eldx < EK || sldx < SK)
    return EXACT_E_ARG;
  if (zero_n < 0 || (zero_n > 0 && !zero)) return EXACT_E_ARG;
  int e = check_chunks(chunk_e, chunk_p0, chunk_n, nchunks, max_chunks, chunk, w_stride, m_stride);
  if (e) return e;
  if (R > 2 || EK % 128 || SK % 128 || (reinterpret_cast<uintptr_t>(ewp) & 15) || (reinterpret_cast<uintptr_t>(swp) & 15))
    return EXACT_E_UNSUPPORTED;
  // the routed experts' split, as exact_gemv_g128_experts_qrow_acc
  const int EG = EK / 128;
  const int64_t enbs = (EN + 63) / 64;
  int64_t ens = (GEMV_WAVES + (int64_t)max_chunks * enbs - 1) / ((int64_t)max_chunks * enbs);
  ens = ens < 1 ? 1 : (ens > EG ? EG : ens);
  const int egmax = (int)((EG + ens - 1) / ens);
  const size_t elds = (size_t)4 * EXPERT_FUSE_CHUNK * egmax * 128 * 2;
  const int64_t etasks = (int64_t)max_chunks * enbs * ens;
  // the shared expert's, as exact_gemv_g128_qrow_acc
  const int SG = SK / 128;
  const int sns = gemv_nsplit(SN, SG);
  const int sgmax = (SG + sns - 1) / sns;
  const size_t slds = (size_t)4 * R * sgmax * 128 * 2;
  const int64_t stasks = (int64_t)((SN + 63) / 64) * sns;
  if (elds > GEMV_XQ_LDS_MAX || slds > GEMV_XQ_LDS_MAX || egmax * 128 > 64 * XQ_LOADS || sgmax * 128 > 64 * XQ_LOADS ||
      enparts > 64 * XQ_PARTS_WIDE || snparts > 64 * XQ_PARTS_WIDE)
    return EXACT_E_UNSUPPORTED;
  const int64_t B1 = (etasks + 3) / 4, B2 = (stasks + 3) / 4;
  if (B1 + B2 > (1LL << 30)) return EXACT_E_UNSUPPORTED;
  const size_t lds = elds > slds ? elds : slds;
  hipStream_t sm = as_stream(stream);
#define QP_GO(VR, W, PLE, PLS)                                                                                         \
  hipLaunchKernelGGL((k_moe_qrow_pair<GEMV_NT != 0, VR, W, PLE, PLS>), dim3((unsigned)(B1 + B2)), dim3(256), lds, sm, exs,  \
                     eldx, epart, enparts, ewp, emp, w_stride, m_stride, chunk_e, chunk_p0, chunk_n, nchunks, et, es_out, EN, \
                     EK, (int)ens, egmax, sxs, sldx, spart, snparts, swp, smp, smh, st, ss_out, R, SN, SK, sns, sgmax, zero,  \
                     zero_n, (int)B1)
#define QP_PLS(VR, W, PLE)                                                                                             \
  do {                                                                                                                 \
    if (snparts <= 64) QP_GO(VR, W, PLE, 1);                                                                           \
    else if (snparts <= 256) QP_GO(VR, W, PLE, 4);                                                                     \
    else QP_GO(VR, W, PLE, XQ_PARTS_WIDE);                                                                             \
  } while (0)
#define QP_PLE(VR, W)                                                                                                  \
  do {                                                                                                                 \
    if (enparts <= 64) QP_PLS(VR, W, 1); else QP_PLS(VR, W, XQ_PARTS_WIDE);                                            \
  } while (0)
  if (smh) {
    if (R == 1) QP_PLE(1, true); else QP_PLE(2, true);
  } else {
    if (R == 1) QP_PLE(1, false); else QP_PLE(2, false);
  }
#undef QP_PLE
#undef QP_PLS
#undef QP_GO
  return launch_status("moe_qrow_pair");
}
