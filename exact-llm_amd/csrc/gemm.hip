// Exact group-128 int8 GEMM for prefill on CDNA4 matrix cores (gfx950).
//
//   t[m][n] = sum_g M[g][n] * sum_{k in g} xq[m][k] * W[n][k]          (SPEC.md:18; GQLin)
//
// Block tile (WM x 64) x (WN x 64): WM x WN waves of 64 x 64 outputs, one 128-wide group per k-step.
//   * Operand tiles move global -> LDS with gfx950's direct loads (global_load_lds_dwordx4: each
//     lane's 16 bytes land at lds_base + 16 * lane), S stages deep, so S - 1 groups are in flight
//     while one is computed. B is the packed weight layout itself (WN 8 KiB tiles per group).
//   * v_mfma_i32_32x32x32_i8 produces the exact int32 group accumulator of each 32 x 32 sub-tile
//     (|acc| < 2^29). The rescale t += acc * M[g][n] is an exact 64-bit integer multiply-add.
//   * Within a group the four sub-tiles of a wave run their MFMA chains one after another; each
//     finished sub-tile's rescale is interleaved with the next sub-tile's chain, so the VALU work
//     and the matrix cores overlap.
// int8 activations (A8): A rows sit row-major in LDS with the 16-byte chunk index XOR-swizzled by
// (row >> 1) & 7 (conflict-free 16-row fragment reads).
// int16 activations (A16, the spec): raw int16 rows in LDS, chunk index XOR-swizzled by row & 15; each
// fragment is split into int8 digits hi = x >> 8 and lo = (x & 255) - 128 (exact_torch.py:101-102)
// and acc = 256 hi.W + lo.W + 128 colsum(W): the hi pass accumulates, is shifted by 8, and the lo pass
// accumulates on top; 128 colsum(W) M is a per-column term added once per group.
//
// Replaces TLinG's fp64 bmm branch (experiments/speed_fair_kaggle.py:739-742) and the cuBLASLt
// torch._int_mm passes of TLin._acc (exact_torch.py:94-119).
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#ifndef GEMM_VALU_PER_MFMA
#define GEMM_VALU_PER_MFMA 4   // VALU instructions the schedule places after each MFMA of a chain
#endif
#ifndef GEMM_PIPE_READS
#define GEMM_PIPE_READS 4      // LDS reads the schedule places in each chain of 4 MFMAs
#endif
#ifndef GEMM_SMALL_M
#define GEMM_SMALL_M 128       // rows up to which the 128-row tile configuration runs
#endif
#ifndef GEMM_SPLIT_TILES
#define GEMM_SPLIT_TILES 128   // split K while the output tiles number fewer than this
#endif

namespace exact {

int zero_bytes(void* dst, int64_t nbytes, hipStream_t st);

// Block = (WM x 64) x (WN x 64): WM x WN waves of 64 x 64 outputs; S LDS stages.
template <int ABITS, int WM, int WN, int S>
struct GemmCfg {
  static constexpr int BM = WM * 64, BN = WN * 64, NT = WN;   // NT packed weight tiles per group
  static constexpr int WAVES = WM * WN, THREADS = WAVES * 64;
  static constexpr int ROWB = ABITS == 15 ? 256 : 128;     // LDS bytes per A row per group
  static constexpr int A_BYTES = BM * ROWB;
  static constexpr int B_BYTES = NT * 8192;
  static constexpr int STAGE = A_BYTES + B_BYTES + 1024;   // + 1 KiB for the BN int16 scales (DMA granule)
  static constexpr int A_KB_PER_WAVE = A_BYTES / 1024 / WAVES;
  static constexpr int B_KB_PER_WAVE = B_BYTES / 1024 / WAVES;
  static constexpr int DMA_PER_GROUP = A_KB_PER_WAVE + B_KB_PER_WAVE;   // per wave (wave 0 issues one more)
  static_assert(S >= 2 && S <= 4, "2 to 4 stages");
  static_assert(A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0, "tiles split evenly over waves");
  static_assert(BN * 2 <= 1024 && NT * 8 <= 64, "scales of one group fit one 1 KiB copy");
};

// LDS byte offset of 16-byte chunk c of A row r
template <int ABITS>
__device__ __forceinline__ int a_off(int r, int c) {
  return ABITS == 15 ? r * 256 + ((c ^ (r & 15)) << 4) : r * 128 + ((c ^ ((r >> 1) & 7)) << 4);
}

// s_waitcnt immediate: vmcnt <= n, expcnt and lgkmcnt not waited on (gfx9 encoding)
#define VMCNT_LE(n) ((((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))

// int16 -> (hi, lo - 128) int8 digits of 16 values held in two 16-byte chunks
__device__ __forceinline__ void split16(v4i p0, v4i p1, v4i& hi, v4i& lo) {
  hi[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x07050301u);
  hi[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x07050301u);
  hi[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x07050301u);
  hi[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x07050301u);
  lo[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x06040200u) ^ 0x80808080;
  lo[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x06040200u) ^ 0x80808080;
  lo[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x06040200u) ^ 0x80808080;
  lo[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x06040200u) ^ 0x80808080;
}

template <int ABITS, int WM, int WN, int S>
__global__ __launch_bounds__(WM * WN * 64, 1) void k_gemm_g128(const void* __restrict__ xv, const int8_t* __restrict__ wp,
                                                      const int16_t* __restrict__ mp, int64_t* __restrict__ t, int M,
                                                      int N, int K, int G, int nbs, int tiles_m, int tiles_n,
                                                      int ksplit, int use_atomic) {
  using C = GemmCfg<ABITS, WM, WN, S>;
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, lh = lane >> 5;

  // XCD-aware order: the blocks of one XCD take consecutive logical tiles (same column block,
  // increasing row block), so each XCD's L2 streams its own slice of the weights once.
  const int nblk = tiles_m * tiles_n * ksplit;
  const int per_xcd = (nblk + 7) / 8;
  const int lb = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (lb >= nblk) return;
  const int kz = lb / (tiles_m * tiles_n);
  const int rem = lb - kz * tiles_m * tiles_n;
  const int bn = rem / tiles_m, bm = rem - bn * tiles_m;
  const int g0 = (int)(((int64_t)kz * G) / ksplit), g1 = (int)(((int64_t)(kz + 1) * G) / ksplit);
  const int row0 = bm * C::BM, nb0 = bn * C::NT;
  const size_t xrow = (size_t)K * (ABITS == 15 ? 2 : 1);
  const int8_t* xb = reinterpret_cast<const int8_t*>(xv);

  // direct global -> LDS copies of group g into stage stg (rows past M / tiles past nbs read a valid
  // neighbour; those outputs are never stored)
  auto issue = [&](int g, int stg) {
    int8_t* sA = smem + stg * C::STAGE;
    int8_t* sB = sA + C::A_BYTES;
#pragma unroll
    for (int i = 0; i < C::A_KB_PER_WAVE; ++i) {
      const int seg = wave * C::A_KB_PER_WAVE + i;          // 1 KiB LDS segment
      int r, c;
      if (ABITS == 15) { r = seg * 4 + (lane >> 4); c = (lane & 15) ^ (r & 15); }
      else { r = seg * 8 + (lane >> 3); c = (lane & 7) ^ ((r >> 1) & 7); }
      const int gr = row0 + r < M ? row0 + r : M - 1;
      const int8_t* src = xb + (size_t)gr * xrow + (size_t)g * C::ROWB + c * 16;
      int8_t* dst = sA + seg * 1024;
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < C::B_KB_PER_WAVE; ++i) {
      const int seg = wave * C::B_KB_PER_WAVE + i;          // tile seg / 8, chunk seg % 8
      const int nb = nb0 + (seg >> 3) < nbs ? nb0 + (seg >> 3) : nbs - 1;
      const int8_t* src = wp + tile_index(nb, g, nbs, G) * 8192 + (seg & 7) * 1024 + lane * 16;
      int8_t* dst = sB + seg * 1024;
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
    if (wave == 0) {   // scales: lanes < 8 NT fetch the tiles' 128-byte rows, the rest refetch into padding
      const int ll = lane % (C::NT * 8);
      const int nb = nb0 + (ll >> 3) < nbs ? nb0 + (ll >> 3) : nbs - 1;
      const int8_t* src = reinterpret_cast<const int8_t*>(mp + tile_index(nb, g, nbs, G) * 64) + (ll & 7) * 16;
      int8_t* dst = sB + C::B_BYTES;
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
  };

  int64_t acc[2][2][16];       // [row sub-tile][col sub-tile][register] running totals
  int64_t colc[2] = {0, 0};    // A16: sum_g 128 colsum_g M_g for the lane's two columns
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[a][b][i] = 0;

  // One group from LDS stage stg: all A / B fragments of the group are read first, then the four
  // 32 x 32 sub-tiles run their MFMA chains one after the other; each finished sub-tile is rescaled
  // (t += acc * M, 64-bit) while the next sub-tile's chain occupies the matrix cores.
  auto group = [&](int stg) {
    const int8_t* sA = smem + stg * C::STAGE;
    const int8_t* sB = sA + C::A_BYTES;
    const int16_t* sM = reinterpret_cast<const int16_t*>(sB + C::B_BYTES);
    v4i bf[2][4], ah[2][4], al[2][4];
    int mcol[2], cs[2] = {0, 0};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int n = wn * 64 + b * 32 + l32;
      mcol[b] = sM[n];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf[b][ks] = *reinterpret_cast<const v4i*>(sB + (n >> 6) * 8192 + (ks * 2 + lh) * 1024 + (n & 63) * 16);
        if (ABITS == 15) {
#pragma unroll
          for (int d = 0; d < 4; ++d) cs[b] = __builtin_amdgcn_sdot4(bf[b][ks][d], 0x01010101, cs[b], false);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int r = wm * 64 + a * 32 + l32;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int ch = ks * 2 + lh;                      // 16-byte int8 chunk of the 128-k group
        if (ABITS == 15) {
          const v4i p0 = *reinterpret_cast<const v4i*>(sA + a_off<15>(r, 2 * ch));
          const v4i p1 = *reinterpret_cast<const v4i*>(sA + a_off<15>(r, 2 * ch + 1));
          split16(p0, p1, ah[a][ks], al[a][ks]);
        } else {
          ah[a][ks] = *reinterpret_cast<const v4i*>(sA + a_off<7>(r, ch));
        }
      }
    }
    // sub-tile t's MFMA chain runs while sub-tile t - 1 is rescaled (the scheduling groups below pin
    // that interleave: one MFMA, then eight VALU instructions of the previous sub-tile's rescale)
    v16i cprev = {};
#pragma unroll
    for (int tile = 0; tile < 5; ++tile) {
      v16i c = {};
      if (tile < 4) {
        const int a = tile >> 1, b = tile & 1;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) c = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah[a][ks], bf[b][ks], c, 0, 0, 0);
        if (ABITS == 15) {
#pragma unroll
          for (int i = 0; i < 16; ++i) c[i] <<= 8;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) c = __builtin_amdgcn_mfma_i32_32x32x32_i8(al[a][ks], bf[b][ks], c, 0, 0, 0);
        }
      }
      if (tile > 0) {
        const int a = (tile - 1) >> 1, b = (tile - 1) & 1;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[a][b][i] += (int64_t)cprev[i] * (int64_t)mcol[b];
      }
      cprev = c;
    }
    // keep every rescale inside this group's block: without a use here the compiler sinks them past
    // the block barrier, where they no longer overlap the matrix-core work
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 16; i += 4)
          asm volatile("" ::"v"(acc[a][b][i]), "v"(acc[a][b][i + 1]), "v"(acc[a][b][i + 2]), "v"(acc[a][b][i + 3]));
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);          // fragment reads
#pragma unroll
    for (int k = 0; k < (ABITS == 15 ? 8 : 4); ++k) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
    for (int t = 1; t < 4; ++t)
#pragma unroll
      for (int k = 0; k < (ABITS == 15 ? 8 : 4); ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // one MFMA of sub-tile t
        __builtin_amdgcn_sched_group_barrier(0x002, ABITS == 15 ? 6 : 8, 0);   // rescale of sub-tile t - 1
      }
    if (ABITS == 15) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int full = cs[b] + __shfl_xor(cs[b], 32, 64);   // the column's other 64 k
        colc[b] += (int64_t)(128 * full) * (int64_t)mcol[b];
      }
    }
  };
  auto wait_next = [&](int g) {   // group g + 1 landed in LDS (later groups may stay in flight); block sync
    const int last = g + S - 1 < g1 - 1 ? g + S - 1 : g1 - 1;
    const int after = last - (g + 1);
    if (after >= 2) __builtin_amdgcn_s_waitcnt(VMCNT_LE(2 * C::DMA_PER_GROUP));
    else if (after == 1) __builtin_amdgcn_s_waitcnt(VMCNT_LE(C::DMA_PER_GROUP));
    else __builtin_amdgcn_s_waitcnt(VMCNT_LE(0));
    // a plain barrier: __syncthreads() would also drain the later groups' copies (a full fence)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  if (g0 < g1) {
#pragma unroll
    for (int i = 0; i < S - 1; ++i)
      if (g0 + i < g1) issue(g0 + i, i);
    wait_next(g0 - 1);
    for (int g = g0; g < g1; ++g) {
      if (g + S - 1 < g1) issue(g + S - 1, (g + S - 1 - g0) % S);
      group((g - g0) % S);
      wait_next(g);
    }
  }

  // C layout of v_mfma_i32_32x32x32_i8: lane l holds column l % 32 and rows 8 (i / 4) + 4 (l / 32) + i % 4
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int col = nb0 * 64 + wn * 64 + b * 32 + l32;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = row0 + wm * 64 + a * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
        if (row < M && col < N) {
          const int64_t val = acc[a][b][i] + colc[b];
          int64_t* dst = t + (size_t)row * N + col;
          if (use_atomic) atomicAdd(reinterpret_cast<unsigned long long*>(dst), (unsigned long long)val);
          else *dst = val;
        }
      }
  }
}

// a copy of x the compiler cannot see through (keeps cheap per-lane arithmetic inside a loop)
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// dword 3 of a raw buffer resource (32-bit untyped data, no swizzle)
#define BUF_DW3 0x00020000
#define LDS __attribute__((address_space(3)))

// s_waitcnt immediate: vmcnt <= vm and lgkmcnt <= lg (gfx9 encoding; expcnt not waited on)
#define WAITCNT(vm, lg) ((((vm) & 15) | (7 << 4) | (((lg) & 15) << 8) | ((((vm) >> 4) & 3) << 14)))

// A8 kernel with the operand fragments software-pipelined across groups. Per wave and group the four
// 32 x 32 sub-tiles run in the order (0,0) (0,1) (1,0) (1,1); each chain of four MFMAs is interleaved
// with the LDS reads the next chains need and with the rescale of the chain before it:
//   chain (0,0): read B1 (this group)       rescale (1,1) of the previous group
//   chain (0,1): read A1 (this group)       rescale (0,0)
//   -- wait until group g + 1 has landed, block barrier, start the copy of group g + S --
//   chain (1,0): read A0 (group g + 1)      rescale (0,1)
//   chain (1,1): read B0 + scales (g + 1)   rescale (1,0)
// so one barrier per group, and every LDS read overlaps matrix-core work.
// WIDE: scales M = mh * 2^15 + mp (mp in [0, 2^15)), both planes copied per group.
// GROUPED (MoE experts): row tile bm is dispatched chunk bm (chunk_e / chunk_p0 / chunk_n, nchunks of them): the
// A rows of pairs chunk_p0 .. + chunk_n (twice as many digit rows with PAIRS) against expert chunk_e's weights at
// wp + e w_stride, mp + e m_stride, colterm + e N; blocks past nchunks exit.
template <int WM, int WN, int S, bool PAIRS, bool WIDE, bool GROUPED = false>
__global__ __launch_bounds__(WM * WN * 64, 1) void k_gemm_a8p(const int8_t* __restrict__ xb, const int8_t* __restrict__ wp,
                                                     const int16_t* __restrict__ mp, const int16_t* __restrict__ mh,
                                                     int64_t* __restrict__ t, int M, int N, int K, int G, int nbs,
                                                     int tiles_m, int tiles_n, int ksplit, int use_atomic,
                                                     const int64_t* __restrict__ colterm, const int32_t* __restrict__ chunk_e,
                                                     const int32_t* __restrict__ chunk_p0, const int32_t* __restrict__ chunk_n,
                                                     const int32_t* __restrict__ nchunks, int64_t w_stride, int64_t m_stride) {
  using C = GemmCfg<7, WM, WN, S>;
  static_assert(EXACT_TILE_GN, "the block's tiles of one group are contiguous in the group-major layout");
  static_assert(C::BN == 128, "one dword copy per lane covers the block's 128 scales");
  constexpr int SMW = WIDE ? 512 : 256;                     // each wave keeps its own copy of the scales
  constexpr int SM_BYTES = C::WAVES * SMW;
  constexpr int STAGE = C::A_BYTES + C::B_BYTES + SM_BYTES;
  constexpr int DPG = C::A_KB_PER_WAVE + C::B_KB_PER_WAVE + (WIDE ? 2 : 1);   // copies per wave per group
  extern __shared__ __attribute__((aligned(1024))) int8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int l32 = lane & 31, lh = lane >> 5;

  const int nblk = tiles_m * tiles_n * ksplit;
  const int per_xcd = (nblk + 7) / 8;
  const int lb = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (lb >= nblk) return;
  const int kz = lb / (tiles_m * tiles_n);
  const int rem = lb - kz * tiles_m * tiles_n;
  const int bn = rem / tiles_m, bm = rem - bn * tiles_m;
  const int g0 = (int)(((int64_t)kz * G) / ksplit), g1 = (int)(((int64_t)(kz + 1) * G) / ksplit);
  const int nb0 = bn * C::NT;
  int row0 = bm * C::BM, Mlim = M;
  if constexpr (GROUPED) {   // uniform over the block: an early exit before any barrier
    if (bm >= nchunks[0]) return;
    const int e = chunk_e[bm];
    const int cn = chunk_n[bm] < (PAIRS ? C::BM / 2 : C::BM) ? chunk_n[bm] : (PAIRS ? C::BM / 2 : C::BM);
    row0 = (PAIRS ? 2 : 1) * chunk_p0[bm];
    Mlim = row0 + (PAIRS ? 2 : 1) * cn;
    if (Mlim > M) Mlim = M;
    wp += (int64_t)e * w_stride;
    mp += (int64_t)e * m_stride;
    if (colterm) colterm += (int64_t)e * N;
  }

  // The per-lane addresses below are recomputed from an opaque copy of the lane id in every group:
  // hoisted out of the loop they would need registers the running totals leave no room for.
  const int ncol = (nbs - nb0) * 64;                        // valid packed columns from nb0 on
  // buffer resources: 32-bit per-lane offsets, the group and the block enter as scalar offsets
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, (int)((uint32_t)M * (uint32_t)K), BUF_DW3);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)wp, (short)0, -1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rM = __builtin_amdgcn_make_buffer_rsrc((void*)mp, (short)0, -1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rMh = __builtin_amdgcn_make_buffer_rsrc((void*)(WIDE ? mh : mp), (short)0, -1, BUF_DW3);
  // per-lane copy offsets, fixed over the groups (the group enters as a scalar offset)
  uint32_t aoffs[C::A_KB_PER_WAVE];
#pragma unroll
  for (int i = 0; i < C::A_KB_PER_WAVE; ++i) {
    const int seg = wave * C::A_KB_PER_WAVE + i;            // 1 KiB LDS segment = 8 rows x 128 bytes
    const int r = seg * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
    const int gr = row0 + r < Mlim ? row0 + r : Mlim - 1;   // rows past the tile's rows read a valid row, never stored
    aoffs[i] = (uint32_t)gr * (uint32_t)K + (uint32_t)(c * 16);
  }
  const int moff = (2 * lane < ncol ? 2 * lane : ncol - 2) * 2;
  auto issue = [&](int g, int stg, int ln) {
    int8_t* sA = smem + stg * STAGE;
    int8_t* sB = sA + C::A_BYTES;
    const int tile0 = g * nbs + nb0;
#pragma unroll
    for (int i = 0; i < C::A_KB_PER_WAVE; ++i) {
      const int seg = wave * C::A_KB_PER_WAVE + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (LDS void*)(sA + seg * 1024), 16, (int)aoffs[i], g * 128, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < C::B_KB_PER_WAVE; ++i) {
      const int seg = wave * C::B_KB_PER_WAVE + i;          // tile seg / 8, 1 KiB chunk seg % 8
      const int tl = nb0 + (seg >> 3) < nbs ? (seg >> 3) : nbs - 1 - nb0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (LDS void*)(sB + seg * 1024), 16, ln * 16,
                                               (tile0 + tl) * 8192 + (seg & 7) * 1024, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rM, (LDS void*)(sB + C::B_BYTES + wave * SMW), 4, moff, tile0 * 128, 0, 0);
    if constexpr (WIDE)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rMh, (LDS void*)(sB + C::B_BYTES + wave * SMW + 256), 4, moff, tile0 * 128, 0,
                                               0);
  };
  // fragment reads; A chunk ks * 2 + lh of row r sits at a_off(r, lh) ^ (ks << 5) (XOR swizzle)
  auto readA = [&](v4i (&f)[4], int stg, int a, int ln) {
    const int off = a_off<7>(wm * 64 + a * 32 + (ln & 31), ln >> 5);
    const int8_t* base = smem + stg * STAGE + (off & ~127);
    const int cb = off & 127;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) f[ks] = *reinterpret_cast<const v4i*>(base + (cb ^ (ks << 5)));
  };
  auto readB = [&](v4i (&f)[4], int stg, int b, int ln) {
    const int8_t* base = smem + stg * STAGE + C::A_BYTES + wn * 8192 + (ln >> 5) * 1024 + (b * 32 + (ln & 31)) * 16;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) f[ks] = *reinterpret_cast<const v4i*>(base + ks * 2048);
  };
  auto readM = [&](int stg, int b, int ln) {
    const int8_t* p = smem + stg * STAGE + C::A_BYTES + C::B_BYTES + wave * SMW + (wn * 64 + b * 32 + (ln & 31)) * 2;
    int m = (int)*reinterpret_cast<const int16_t*>(p);
    if constexpr (WIDE) m |= (int)*reinterpret_cast<const int16_t*>(p + 256) << 15;
    return m;
  };
  auto chain = [&](const v4i (&a)[4], const v4i (&b)[4]) {
    v16i c = {};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ks], b[ks], c, 0, 0, 0);
    return c;
  };
  // PAIRS: one running total per output row pair (256 hi + lo fits int32 per group: 2^29 + 2^21)
  constexpr int NT_ = PAIRS ? 8 : 16;
  int64_t acc[2][2][NT_];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < NT_; ++i) acc[a][b][i] = 0;
  // t += c * m, pinned in place: without a use here the compiler sinks the multiply-adds past the next
  // barrier, where they no longer overlap the matrix-core work
  auto rescale = [&](int64_t (&ac)[NT_], const v16i& c, int m_) {
    const int m = opaque(m_);   // a plain 32-bit value here, so each product is one v_mad_i64_i32
    if constexpr (PAIRS) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = 2 * j;   // i % 4 in {0, 2}: rows 2r (hi) and 2r + 1 (lo) at i and i + 1
        ac[j] += (int64_t)((c[i] << 8) + c[i + 1]) * (int64_t)m;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) ac[i] += (int64_t)c[i] * (int64_t)m;
    }
#pragma unroll
    for (int i = 0; i < NT_; i += 4) asm volatile("" ::"v"(ac[i]), "v"(ac[i + 1]), "v"(ac[i + 2]), "v"(ac[i + 3]));
  };
  // one chain of 4 MFMAs interleaved with `reads` LDS reads and the 16 rescale multiply-adds
#define PIPE_PATTERN(reads)                                                                    \
  do {                                                                                         \
    _Pragma("unroll") for (int k_ = 0; k_ < 4; ++k_) {                                         \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                       \
      if (k_ < (reads)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                      \
      __builtin_amdgcn_sched_group_barrier(0x002, GEMM_VALU_PER_MFMA, 0);                      \
    }                                                                                          \
  } while (0)

  if (g0 < g1) {
    const int nst = g1 - g0 < S ? g1 - g0 : S;
    for (int i = 0; i < nst; ++i) issue(g0 + i, i, opaque(lane));
    // group g0 landed: the later groups' copies may stay in flight
    if (nst >= 4) __builtin_amdgcn_s_waitcnt(WAITCNT(3 * DPG, 15));
    else if (nst == 3) __builtin_amdgcn_s_waitcnt(WAITCNT(2 * DPG, 15));
    else if (nst == 2) __builtin_amdgcn_s_waitcnt(WAITCNT(DPG, 15));
    else __builtin_amdgcn_s_waitcnt(WAITCNT(0, 15));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    v4i A0[4], B0[4], A1[4], B1[4];
    readA(A0, 0, 0, lane);
    readB(B0, 0, 0, lane);
    int m0 = readM(0, 0, lane), m1 = readM(0, 1, lane);
    v16i cp = {};
    int mprev = 0;
    int stg = 0;
    for (int g = g0; g < g1; ++g) {
      const int ln = lane;
      const int nstg = stg + 1 == S ? 0 : stg + 1;
      readB(B1, stg, 1, ln);
      const v16i c00 = chain(A0, B0);
      rescale(acc[1][1], cp, mprev);
      PIPE_PATTERN(GEMM_PIPE_READS);
      __builtin_amdgcn_sched_barrier(0);
      readA(A1, stg, 1, ln);
      const v16i c01 = chain(A0, B1);
      rescale(acc[0][0], c00, m0);
      PIPE_PATTERN(GEMM_PIPE_READS);
      // all of this wave's reads of stage stg are done; group g + 1 has landed; then stage stg is
      // free for group g + S
      const int ahead = (g1 - 1 < g + S - 1 ? g1 - 1 : g + S - 1) - (g + 1);   // groups in flight after g + 1
      if (ahead >= 2) __builtin_amdgcn_s_waitcnt(WAITCNT(2 * DPG, 0));
      else if (ahead == 1) __builtin_amdgcn_s_waitcnt(WAITCNT(DPG, 0));
      else __builtin_amdgcn_s_waitcnt(WAITCNT(0, 0));
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (g + S < g1) issue(g + S, stg, ln);
      readA(A0, nstg, 0, ln);
      const v16i c10 = chain(A1, B0);
      rescale(acc[0][1], c01, m1);
      PIPE_PATTERN(GEMM_PIPE_READS);
      __builtin_amdgcn_sched_barrier(0);
      readB(B0, nstg, 0, ln);
      const int mn0 = readM(nstg, 0, ln), mn1 = readM(nstg, 1, ln);
      const v16i c11 = chain(A1, B1);
      rescale(acc[1][0], c10, m0);
      PIPE_PATTERN(GEMM_PIPE_READS);
      cp = c11;
      mprev = m1;
      m0 = mn0;
      m1 = mn1;
      stg = nstg;
    }
    rescale(acc[1][1], cp, mprev);
  }
#undef PIPE_PATTERN

  if constexpr (PAIRS) {
    // A16 as digit rows: rows 2r (hi = x >> 8) and 2r + 1 (lo = (x & 255) - 128) of the A operand come from
    // activation row r and sit in one lane at i and i + 1 (i % 4 in {0, 2}); the rescale combined them per
    // group, so t[r] = sum_g (256 hi_g + lo_g) M_g + 128 sum_g colsum_g M_g (exact_torch.py:101-102), colterm
    // = the last sum.
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int col = nb0 * 64 + wn * 64 + b * 32 + l32;
      const int64_t ct = (kz == 0 && col < N) ? 128 * colterm[col] : 0;
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const int row = row0 + wm * 64 + a * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);   // even
          if (row < Mlim && col < N) {
            const int64_t val = acc[a][b][i >> 1] + ct;
            int64_t* dst = t + (size_t)(row >> 1) * N + col;
            if (use_atomic) atomicAdd(reinterpret_cast<unsigned long long*>(dst), (unsigned long long)val);
            else *dst = val;
          }
        }
    }
  } else {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int col = nb0 * 64 + wn * 64 + b * 32 + l32;
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = row0 + wm * 64 + a * 32 + 8 * (i >> 2) + 4 * lh + (i & 3);
          if (row < Mlim && col < N) {
            const int64_t val = acc[a][b][i];
            int64_t* dst = t + (size_t)row * N + col;
            if (use_atomic) atomicAdd(reinterpret_cast<unsigned long long*>(dst), (unsigned long long)val);
            else *dst = val;
          }
        }
    }
  }
}

}  // namespace exact
#include "../_build/gemm_asm.inc"
namespace exact {

// The A8 GEMM (and A16 as digit-row pairs) with its main loop in generated assembly (gen_gemm_asm.py, which states
// the schedule and the register map): 256 x 128 tiles (128 x 128 output rows x columns for PAIRS), one K pass, plain
// stores. This function computes the block's tile, every per-lane copy / read / store offset and the scalar state,
// and hands them to the asm in pinned registers. Mrows: rows of the A operand (digit rows for PAIRS); tiles past
// M or N (ragged edges) store under a lane mask; A rows past Mrows read row Mrows - 1 (never stored).
template <bool PAIRS>
__global__ __launch_bounds__(512, 1) void k_gemm_asm(const int8_t* __restrict__ xb, const int8_t* __restrict__ wp,
                                                     const int16_t* __restrict__ mp, int64_t* __restrict__ t,
                                                     const int64_t* __restrict__ colterm, int Mrows, int N, int K, int G,
                                                     int nbs, int tiles_m, int tiles_n) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int j = lane & 15, q = lane >> 4;
  // XCD-aware order as k_gemm_a8p: the blocks of one XCD take consecutive tiles (one column block, its row blocks)
  const int nblk = tiles_m * tiles_n;
  const int per_xcd = (nblk + 7) / 8;
  const int lb = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (lb >= nblk) return;
  const int bn = lb / tiles_m, bm = lb - bn * tiles_m;
  const int row0 = bm * 256, nb0 = bn * 2, col0 = nb0 * 64;
  const int g0 = 0, g1 = G;
  const int iters = __builtin_amdgcn_readfirstlane((g1 - g0 + 5) / 6);
  const int phase = __builtin_amdgcn_readfirstlane(6 * iters - (g1 - g0));
  // copy offsets: A segment i of this wave = rows 8 (4 wave + i) + lane / 8, chunk slot lane % 8 holding the row's
  // 16-byte chunk (lane % 8) ^ ((row >> 1) & 7)
  uint32_t vad[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (wave * 4 + i) * 8 + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
    const int gr = row0 + r < Mrows ? row0 + r : Mrows - 1;
    vad[i] = (uint32_t)gr * (uint32_t)K + (uint32_t)(c * 16);
  }
  // B: LDS slot 16 cs + j of each 1 KiB chunk holds column 4 j + cs of the packed tile
  const int vbdma = (4 * (lane & 15) + (lane >> 4)) * 16;
  int bc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int seg = wave * 2 + i;
    const int tl = nb0 + (seg >> 3) < nbs ? (seg >> 3) : nbs - 1 - nb0;   // a missing second tile reads the first
    bc[i] = (nb0 + tl) * 8192 + (seg & 7) * 1024;
  }
  const int ncol = (nbs - nb0) * 64;
  const int vmdma = (2 * lane < ncol ? 2 * lane : ncol - 2) * 2;
  // LDS read bases (the asm adds stage, sub-tile and k-half offsets as immediates)
  int vard[4];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    vard[kh] = wm * 8192 + j * 128 + (((kh * 4 + q) ^ ((j >> 1) & 7)) << 4);
    vard[2 + kh] = vard[kh] + GEMM_ASM_A_HI;
  }
  const int vbrd = GEMM_ASM_B_BASE + wn * 8192 + q * 1024 + j * 16;
  const int vmrd = GEMM_ASM_M_BASE + wave * 256 + wn * 128 + 8 * j;
  // outputs: the lane's first row (4 rows, or 2 output rows of digit-row pairs, per 16-row sub-tile) and 4 columns
  const int Mout = PAIRS ? Mrows / 2 : Mrows;
  const int orow = PAIRS ? row0 / 2 + wm * 32 + 2 * q : row0 + wm * 64 + 4 * q;
  const int ocol = col0 + wn * 64 + 4 * j;
  const int vst = (int)(((uint32_t)orow * (uint32_t)N + (uint32_t)ocol) * 8u);
  const int full =
      __builtin_amdgcn_readfirstlane(((PAIRS ? row0 / 2 + 128 <= Mout : row0 + 256 <= Mrows) && col0 + 128 <= N) ? 1 : 0);
  const __amdgpu_buffer_rsrc_t rA =
      __builtin_amdgcn_make_buffer_rsrc((void*)xb, (short)0, (int)((uint32_t)Mrows * (uint32_t)K), BUF_DW3);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc((void*)wp, (short)0, -1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rM = __builtin_amdgcn_make_buffer_rsrc((void*)mp, (short)0, -1, BUF_DW3);
  const __amdgpu_buffer_rsrc_t rT = __builtin_amdgcn_make_buffer_rsrc((void*)t, (short)0, -1, BUF_DW3);
  const int asoff = g0 * 128, bg = g0 * nbs * 8192, mg = (g0 * nbs + nb0) * 128;
  const int wavea = wave * 4096, waveb = GEMM_ASM_B_BASE + wave * 2048, wavem = GEMM_ASM_M_BASE + wave * 256;
  if constexpr (PAIRS) {
    const __amdgpu_buffer_rsrc_t rCt = __builtin_amdgcn_make_buffer_rsrc((void*)colterm, (short)0, -1, BUF_DW3);
    const int ctoff = (ocol < N ? ocol : 0) * 8;
    gemm_asm_main_pairs(g0, g1, iters, phase, full, asoff, bg, bc[0], bc[1], mg, nbs * 8192, nbs * 128, wavea, waveb,
                        wavem, N * 8, Mout, N, rA, rB, rM, rT, (int)vad[0], (int)vad[1], (int)vad[2], (int)vad[3], vbdma,
                        vmdma, vard[0], vard[1], vard[2], vard[3], vbrd, vmrd, vst, orow, ocol, rCt, ctoff);
  } else {
    gemm_asm_main_a8(g0, g1, iters, phase, full, asoff, bg, bc[0], bc[1], mg, nbs * 8192, nbs * 128, wavea, waveb, wavem,
                     N * 8, Mout, N, rA, rB, rM, rT, (int)vad[0], (int)vad[1], (int)vad[2], (int)vad[3], vbdma, vmdma,
                     vard[0], vard[1], vard[2], vard[3], vbrd, vmrd, vst, orow, ocol);
  }
}

// int16 rows -> interleaved int8 digit rows: x8[2r] = x[r] >> 8, x8[2r + 1] = (x[r] & 255) - 128.
// 16 values per thread; K % 16 == 0.
__global__ __launch_bounds__(256) void k_split_rows_a16(const int16_t* __restrict__ x, int8_t* __restrict__ x8, int64_t M,
                                                        int K, const int32_t* __restrict__ row_map = nullptr) {
  const int64_t n16 = M * (K / 16);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / (K / 16), c = (i - r * (K / 16)) * 16;
    const v4i* src = reinterpret_cast<const v4i*>(x + (row_map ? (int64_t)row_map[r] : r) * K + c);
    const v4i p0 = src[0], p1 = src[1];
    v4i hi, lo;
    hi[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x07050301u);
    hi[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x07050301u);
    hi[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x07050301u);
    hi[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x07050301u);
    lo[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x06040200u) ^ 0x80808080;
    lo[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x06040200u) ^ 0x80808080;
    lo[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x06040200u) ^ 0x80808080;
    lo[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x06040200u) ^ 0x80808080;
    *reinterpret_cast<v4i*>(x8 + (2 * r) * K + c) = hi;
    *reinterpret_cast<v4i*>(x8 + (2 * r + 1) * K + c) = lo;
  }
}

// gathered int8 rows: x8[p] = x[row_map[p]] (16 bytes per thread; K % 16 == 0)
__global__ __launch_bounds__(256) void k_gather_rows_a8(const int8_t* __restrict__ x, int8_t* __restrict__ x8, int64_t P, int K,
                                                        const int32_t* __restrict__ row_map) {
  const int64_t n16 = P * (K / 16);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = i / (K / 16), c = (i - p * (K / 16)) * 16;
    *reinterpret_cast<v4i*>(x8 + p * K + c) = *reinterpret_cast<const v4i*>(x + (int64_t)row_map[p] * K + c);
  }
}

template <int ABITS, int WM, int WN, int S>
static int gemm_launch(const void* x, const int8_t* wp, const int16_t* mp, int64_t* t, int M, int N, int K,
                       hipStream_t st, int ksplit_req, bool zeroed = false) {
  using C = GemmCfg<ABITS, WM, WN, S>;
  static bool attr_set = false;
  const size_t lds = S * (size_t)C::STAGE;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_g128<ABITS, WM, WN, S>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr_set = true;
  }
  const int G = K / 128, nbs = (N + 63) / 64;
  const int tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (nbs + C::NT - 1) / C::NT;
  int ksplit = ksplit_req;
  if (ksplit <= 0) {   // split K only when the output tiles fill fewer than half the 256 CUs (the split costs a
                       // zero fill and 64-bit atomics on t, more than a partly idle chip)
    ksplit = 1;
    while (tiles_m * tiles_n * ksplit < GEMM_SPLIT_TILES && G / (ksplit * 2) >= 8) ksplit *= 2;
  }
  if (ksplit > G) ksplit = G;
  const int use_atomic = ksplit > 1;
  if (use_atomic && !zeroed) {
    int e = zero_bytes(t, (int64_t)M * N * 8, st);
    if (e) return e;
  }
  const int nblk = tiles_m * tiles_n * ksplit;
  const int grid = ((nblk + 7) / 8) * 8;
  hipLaunchKernelGGL((k_gemm_g128<ABITS, WM, WN, S>), dim3(grid), dim3(C::THREADS), lds, st, x, wp, mp, t, M, N, K, G, nbs,
                     tiles_m, tiles_n, ksplit, use_atomic);
  return launch_status("gemm_g128");
}

#ifndef GEMM_KSPLIT
#define GEMM_KSPLIT 0
#endif
// (waves along M, waves along N, LDS stages)
#ifndef GEMM_A8_CFG
#define GEMM_A8_CFG 4, 2, 2
#endif
#ifndef GEMM_A16_CFG
#define GEMM_A16_CFG 2, 2, 3
#endif

#ifndef GEMM_A8P_CFG
#define GEMM_A8P_CFG 4, 2, 3
#endif

#ifndef GEMM_ASM
#define GEMM_ASM 1
#endif

// M: rows of the A operand (digit rows for PAIRS); one K pass, t fully overwritten
template <bool PAIRS>
static int gemm_launch_asm(const int8_t* x, const int8_t* wp, const int16_t* mp, int64_t* t, const int64_t* colterm, int M,
                           int N, int K, hipStream_t st) {
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_asm<PAIRS>), hipFuncAttributeMaxDynamicSharedMemorySize,
                              GEMM_ASM_LDS_BYTES);
    attr_set = true;
  }
  const int G = K / 128, nbs = (N + 63) / 64;
  const int tiles_m = (M + 255) / 256, tiles_n = (nbs + 1) / 2;
  const int nblk = tiles_m * tiles_n;
  const int grid = ((nblk + 7) / 8) * 8;
  hipLaunchKernelGGL(k_gemm_asm<PAIRS>, dim3(grid), dim3(512), GEMM_ASM_LDS_BYTES, st, x, wp, mp, t, colterm, M, N, K, G,
                     nbs, tiles_m, tiles_n);
  return launch_status("gemm_g128");
}

// M: rows of the A operand (digit rows when PAIRS: the output has M / 2 rows, written through colterm)
template <int WM, int WN, int S, bool PAIRS, bool WIDE>
static int gemm_launch_a8p_t(const void* x, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int M, int N,
                             int K, hipStream_t st, int ksplit_req, const int64_t* colterm, bool zeroed) {
  using C = GemmCfg<7, WM, WN, S>;
  static bool attr_set = false;
  const size_t lds = S * (size_t)(C::A_BYTES + C::B_BYTES + C::WAVES * (WIDE ? 512 : 256));
  static_assert(S * (C::A_BYTES + C::B_BYTES + C::WAVES * (WIDE ? 512 : 256)) <= 160 * 1024, "fits the 160 KiB LDS");
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_a8p<WM, WN, S, PAIRS, WIDE>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr_set = true;
  }
  const int G = K / 128, nbs = (N + 63) / 64;
  const int tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (nbs + C::NT - 1) / C::NT;
  int ksplit = ksplit_req;
  if (ksplit <= 0) {
    ksplit = 1;
    while (tiles_m * tiles_n * ksplit < GEMM_SPLIT_TILES && G / (ksplit * 2) >= 8) ksplit *= 2;
  }
  if (ksplit > G) ksplit = G;
  // one K pass over enough tiles: the assembly main loop (same tiles and outputs; 32-bit offsets into x, W and t)
  if (GEMM_ASM && ksplit == 1 && !WIDE && WM == 4 && WN == 2 &&
      (int64_t)(PAIRS ? M / 2 : M) * N * 8 < (1LL << 32) && (int64_t)G * nbs * 8192 < (1LL << 32))
    return gemm_launch_asm<PAIRS>(reinterpret_cast<const int8_t*>(x), wp, mp, t, colterm, M, N, K, st);
  const int use_atomic = ksplit > 1;
  if (use_atomic && !zeroed) {
    int e = zero_bytes(t, (int64_t)(PAIRS ? M / 2 : M) * N * 8, st);
    if (e) return e;
  }
  const int nblk = tiles_m * tiles_n * ksplit;
  const int grid = ((nblk + 7) / 8) * 8;
  hipLaunchKernelGGL((k_gemm_a8p<WM, WN, S, PAIRS, WIDE>), dim3(grid), dim3(C::THREADS), lds, st,
                     reinterpret_cast<const int8_t*>(x), wp, mp, mh, t, M, N, K, G, nbs, tiles_m, tiles_n, ksplit, use_atomic,
                     colterm, nullptr, nullptr, nullptr, nullptr, (int64_t)0, (int64_t)0);
  return launch_status("gemm_g128");
}

// MoE experts: one grouped launch over the dispatched chunks (row tile = chunk), max_chunks row tiles
template <int WM, int WN, int S, bool PAIRS>
static int gemm_launch_experts(const int8_t* x8, const int8_t* wp, const int16_t* mp, int64_t w_stride, int64_t m_stride,
                               const int64_t* colterm, const int32_t* chunk_e, const int32_t* chunk_p0,
                               const int32_t* chunk_n, const int32_t* nchunks, int max_chunks, int64_t* t, int M, int N,
                               int K, hipStream_t st) {
  using C = GemmCfg<7, WM, WN, S>;
  static bool attr_set = false;
  const size_t lds = S * (size_t)(C::A_BYTES + C::B_BYTES + C::WAVES * 256);
  if (!attr_set) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_a8p<WM, WN, S, PAIRS, false, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    attr_set = true;
  }
  const int G = K / 128, nbs = (N + 63) / 64;
  const int tiles_n = (nbs + C::NT - 1) / C::NT;
  const int nblk = max_chunks * tiles_n;
  const int grid = ((nblk + 7) / 8) * 8;
  hipLaunchKernelGGL((k_gemm_a8p<WM, WN, S, PAIRS, false, true>), dim3(grid), dim3(C::THREADS), lds, st, x8, wp, mp, nullptr, t,
                     M, N, K, G, nbs, max_chunks, tiles_n, 1, 0, colterm, chunk_e, chunk_p0, chunk_n, nchunks, w_stride,
                     m_stride);
  return launch_status("gemm_g128_experts");
}

template <int WM, int WN, int S, bool PAIRS = false>
static int gemm_launch_a8p(const void* x, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int M, int N,
                           int K, hipStream_t st, int ksplit_req, const int64_t* colterm = nullptr, bool zeroed = false) {
  // up to 128 rows (prompts of 49-64 tokens as int16 digit rows): 128-row tiles, two 4-wave blocks per CU, instead
  // of 256-row tiles half of padding
  if (M <= GEMM_SMALL_M && WM != 2) {
    if (mh) return gemm_launch_a8p_t<2, WN, 2, PAIRS, true>(x, wp, mp, mh, t, M, N, K, st, ksplit_req, colterm, zeroed);
    return gemm_launch_a8p_t<2, WN, 2, PAIRS, false>(x, wp, mp, nullptr, t, M, N, K, st, ksplit_req, colterm, zeroed);
  }
  if (mh) return gemm_launch_a8p_t<WM, WN, S, PAIRS, true>(x, wp, mp, mh, t, M, N, K, st, ksplit_req, colterm, zeroed);
  return gemm_launch_a8p_t<WM, WN, S, PAIRS, false>(x, wp, mp, nullptr, t, M, N, K, st, ksplit_req, colterm, zeroed);
}

#ifndef GEMM_A8P
#define GEMM_A8P 1
#endif

// Wide scales (mh) run on the A8 kernel only: int8 rows with M K < 2^32 (int16 rows take exact_gemm_g128_a16).
// zeroed: t holds zeros on entry, so a K split adds into it without a clear launch.
int gemm_mfma(const void* x, int abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int M, int N,
              int K, hipStream_t st, bool zeroed) {
  const bool a8p = GEMM_A8P && abits == 7 && (int64_t)M * K < (1LL << 32);
  if (mh && !a8p) return EXACT_E_UNSUPPORTED;
  if (abits == 15) return gemm_launch<15, GEMM_A16_CFG>(x, wp, mp, t, M, N, K, st, GEMM_KSPLIT, zeroed);
  if (a8p) return gemm_launch_a8p<GEMM_A8P_CFG>(x, wp, mp, mh, t, M, N, K, st, GEMM_KSPLIT, nullptr, zeroed);
  return gemm_launch<7, GEMM_A8_CFG>(x, wp, mp, t, M, N, K, st, GEMM_KSPLIT, zeroed);
}

int gemv_launch(const void* x, int abits, const int8_t* wp, const int16_t* mp, const int16_t* mh, int64_t* t, int R, int N,
                int K, hipStream_t st, bool accumulate, const int64_t* colterm);

// int16 rows with colterm: up to A16_GEMV_CHUNKS_MAX x 16 rows as GEMV row chunks (one weight stream per chunk, no
// all-ones row needed), more rows as interleaved digit rows on the A8 GEMM, which streams the weights once. 7B prefill
// (ms, graph replays): 32 tokens 5.47 and 48 tokens 7.74 as 2 and 3 chunks, 49 tokens 4.60 on the GEMM.
#ifndef A16_GEMV_CHUNKS_MAX
#define A16_GEMV_CHUNKS_MAX 1
#endif
int gemm_a16_digit_rows(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh, const int64_t* colterm,
                        int8_t* x8, int64_t* t, int M, int N, int K, hipStream_t st, bool zeroed) {
  if (M <= A16_GEMV_CHUNKS_MAX * 16) {
    for (int r0 = 0; r0 < M; r0 += 16) {
      const int rows = M - r0 < 16 ? M - r0 : 16;
      int e = gemv_launch(x + (size_t)r0 * K, 15, wp, mp, mh, t + (size_t)r0 * N, rows, N, K, st, zeroed, colterm);
      if (e) return e;
    }
    return EXACT_OK;
  }
  const int64_t n16 = (int64_t)M * (K / 16);
  const int blocks = (int)std::min<int64_t>((n16 + 255) / 256, 8192);
  hipLaunchKernelGGL(k_split_rows_a16, dim3(blocks), dim3(256), 0, st, x, x8, (int64_t)M, K, nullptr);
  return gemm_launch_a8p<GEMM_A8P_CFG, true>(x8, wp, mp, mh, t, 2 * M, N, K, st, GEMM_KSPLIT, colterm, zeroed);
}

}  // namespace exact

using namespace exact;

// pairs per dispatched chunk the experts GEMM takes: one 256-row tile (128 pairs as digit-row pairs)
#define EXPERT_CHUNK_A16 128
#define EXPERT_CHUNK_A8 256

extern "C" int exact_gemm_g128_experts(const void* x, int32_t abits, const int32_t* row_map, const int8_t* wp, const int16_t* mp,
                                       int64_t w_stride, int64_t m_stride, const int64_t* colterm, int8_t* x8,
                                       const int32_t* chunk_e, const int32_t* chunk_p0, const int32_t* chunk_n,
                                       const int32_t* nchunks, int32_t max_chunks, int64_t* t, int32_t P, int32_t N, int32_t K,
                                       void* stream) {
  if (!x || !wp || !mp || !x8 || !chunk_e || !chunk_p0 || !chunk_n || !nchunks || !t) return EXACT_E_ARG;
  if (P <= 0 || N <= 0 || K <= 0 || max_chunks <= 0 || w_stride <= 0 || m_stride <= 0) return EXACT_E_ARG;
  if (abits == 15 && !colterm) return EXACT_E_ARG;
  if ((abits != 15 && abits != 7) || K % 128 || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(x8) & 15) ||
      (reinterpret_cast<uintptr_t>(wp) & 15) || (w_stride & 15))
    return EXACT_E_UNSUPPORTED;
  const int64_t rows = (abits == 15 ? 2 : 1) * (int64_t)P;
  if (rows * K >= (1LL << 32)) return EXACT_E_UNSUPPORTED;   // 32-bit buffer offsets
  hipStream_t st = as_stream(stream);
  const int64_t n16 = (int64_t)P * (K / 16);
  const int blocks = (int)std::min<int64_t>((n16 + 255) / 256, 8192);
  if (abits == 15) {
    hipLaunchKernelGGL(k_split_rows_a16, dim3(blocks), dim3(256), 0, st, static_cast<const int16_t*>(x), x8, (int64_t)P, K,
                       row_map);
    return gemm_launch_experts<GEMM_A8P_CFG, true>(x8, wp, mp, w_stride, m_stride, colterm, chunk_e, chunk_p0, chunk_n,
                                                   nchunks, max_chunks, t, (int)rows, N, K, st);
  }
  const int8_t* xa = static_cast<const int8_t*>(x);
  if (row_map) {
    hipLaunchKernelGGL(k_gather_rows_a8, dim3(blocks), dim3(256), 0, st, xa, x8, (int64_t)P, K, row_map);
    xa = x8;
  }
  return gemm_launch_experts<GEMM_A8P_CFG, false>(xa, wp, mp, w_stride, m_stride, nullptr, chunk_e, chunk_p0, chunk_n, nchunks,
                                                  max_chunks, t, (int)rows, N, K, st);
}

static int gemm_a16_entry(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                          const int64_t* colterm, int8_t* x8, int64_t* t, int32_t R, int32_t N, int32_t K, void* stream,
                          bool zeroed) {
  if (!x || !wp || !mp || !colterm || !x8 || !t || R <= 0 || N <= 0 || K <= 0) return EXACT_E_ARG;
  if (K % 128 || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(x8) & 15) ||
      (reinterpret_cast<uintptr_t>(wp) & 15))
    return EXACT_E_UNSUPPORTED;
  if (2 * (int64_t)R * K >= (1LL << 32)) return EXACT_E_UNSUPPORTED;   // 32-bit buffer offsets of the digit rows
  return gemm_a16_digit_rows(x, wp, mp, mh, colterm, x8, t, R, N, K, as_stream(stream), zeroed);
}

extern "C" int exact_gemm_g128_a16(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                   const int64_t* colterm, int8_t* x8, int64_t* t, int32_t R, int32_t N, int32_t K,
                                   void* stream) {
  return gemm_a16_entry(x, wp, mp, mh, colterm, x8, t, R, N, K, stream, false);
}

extern "C" int exact_gemm_g128_a16_zeroed(const int16_t* x, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                          const int64_t* colterm, int8_t* x8, int64_t* t, int32_t R, int32_t N, int32_t K,
                                          void* stream) {
  return gemm_a16_entry(x, wp, mp, mh, colterm, x8, t, R, N, K, stream, true);
}

extern "C" int exact_gemm_g128_digits(const int8_t* x8, const int8_t* wp, const int16_t* mp, const int16_t* mh,
                                      const int64_t* colterm, int64_t* t, int32_t R, int32_t N, int32_t K, int32_t zeroed,
                                      void* stream) {
  if (!x8 || !wp || !mp || !colterm || !t || R <= 0 || N <= 0 || K <= 0) return EXACT_E_ARG;
  if (K % 128 || (reinterpret_cast<uintptr_t>(x8) & 15) || (reinterpret_cast<uintptr_t>(wp) & 15)) return EXACT_E_UNSUPPORTED;
  if (2 * (int64_t)R * K >= (1LL << 32)) return EXACT_E_UNSUPPORTED;   // 32-bit buffer offsets of the digit rows
  return gemm_launch_a8p<GEMM_A8P_CFG, true>(x8, wp, mp, mh, t, 2 * R, N, K, as_stream(stream), GEMM_KSPLIT, colterm,
                                             zeroed != 0);
}
