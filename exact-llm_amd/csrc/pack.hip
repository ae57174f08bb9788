// Weight packing, the seeded synthetic integer artifact, and the Q16 embedding table.
//
// Packed linear layout (N outputs, K inputs, G = K/128, nbs = ceil(N/64), T = tile_index(nb, g)):
//   wp[(T*8 + j)*1024 + l*16 + b] = W[n = nb*64 + l][k = g*128 + j*16 + b]
//   mp[T*64 + l]                  = M[g][n]
// so the 64 x 128 tile (nb, g) is 8 KiB of contiguous bytes: the decode GEMV streams it with
// 16-byte loads and hands it to the matrix cores without any reshuffle. A buffer may hold several
// linears with the same K stacked along the output rows (fused q|k|v, gate|up); each part starts on
// a 64-row boundary and is written with its own row offset.
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace exact {

// one thread per 16-byte (row, 16-k) chunk of the packed tile array
__global__ void k_synth_w(uint64_t key, const uint32_t* __restrict__ thr, int8_t* __restrict__ wp, int N, int K, int G,
                          int64_t nchunks, int nb_off, int64_t nbs_tot) {
  __shared__ uint32_t th[256];
  for (int i = threadIdx.x; i < 254; i += blockDim.x) th[i] = thr[i];
  __syncthreads();
  for (int64_t ch = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; ch < nchunks; ch += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(ch & 63);
    const int j = (int)((ch >> 6) & 7);
    const int64_t lt = ch >> 9;            // part-local tile, (nb, g) with g fastest
    const int g = (int)(lt % G);
    const int64_t nb = lt / G;
    const int64_t n = nb * 64 + l;
    const int64_t tile = tile_index(nb + nb_off, g, nbs_tot, G);
    uint32_t wd[4] = {0, 0, 0, 0};
    if (n < N) {
      const uint64_t base = (uint64_t)n * K + (uint64_t)g * 128 + j * 16;
      for (int b = 0; b < 16; ++b) {
        const uint32_t u = (uint32_t)(splitmix64(key, base + b) >> 32);
        int lo = 0, hi = 254;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (th[mid] <= u) lo = mid + 1; else hi = mid;
        }
        const uint32_t w = (uint32_t)(uint8_t)(int8_t)(lo - 127);
        wd[b >> 2] |= w << (8 * (b & 3));
      }
    }
    v4i o = {(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
    *reinterpret_cast<v4i*>(wp + (tile * 8 + j) * 1024 + l * 16) = o;
  }
}

__global__ void k_synth_m(uint64_t key, int32_t lo, int32_t hi, int16_t* __restrict__ mp, int N, int G, int64_t total,
                          int nb_off, int64_t nbs_tot) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t lt = i >> 6;
    const int g = (int)(lt % G);
    const int64_t nb = lt / G;
    const int64_t n = nb * 64 + l;
    int16_t m = 0;
    if (n < N) {
      const uint64_t u = splitmix64(key, (uint64_t)n * G + g) >> 32;
      m = (int16_t)(lo + (int32_t)((u * (uint64_t)(hi - lo)) >> 32));
    }
    mp[tile_index(nb + nb_off, g, nbs_tot, G) * 64 + l] = m;
  }
}

__global__ void k_synth_vec(uint64_t key, int64_t lo, uint64_t span, int64_t* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t u = splitmix64(key, (uint64_t)i) >> 32;
    out[i] = lo + (int64_t)((u * span) >> 32);
  }
}

__global__ void k_pack(const int8_t* __restrict__ w, const int16_t* __restrict__ m, int8_t* __restrict__ wp,
                       int16_t* __restrict__ mp, int N, int K, int G, int64_t nchunks, int nb_off, int64_t nbs_tot) {
  for (int64_t ch = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; ch < nchunks; ch += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(ch & 63);
    const int j = (int)((ch >> 6) & 7);
    const int64_t lt = ch >> 9;
    const int g = (int)(lt % G);
    const int64_t nb = lt / G;
    const int64_t n = nb * 64 + l;
    const int64_t tile = tile_index(nb + nb_off, g, nbs_tot, G);
    uint32_t wd[4] = {0, 0, 0, 0};
    if (n < N) {
      const int64_t k0 = (int64_t)g * 128 + j * 16;
      for (int b = 0; b < 16; ++b) wd[b >> 2] |= (uint32_t)(uint8_t)w[(k0 + b) * N + n] << (8 * (b & 3));
      if (j == 0) mp[tile * 64 + l] = m[(int64_t)g * N + n];
    } else if (j == 0) {
      mp[tile * 64 + l] = 0;
    }
    v4i o = {(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
    *reinterpret_cast<v4i*>(wp + (tile * 8 + j) * 1024 + l * 16) = o;
  }
}

// scales only: mp[tile * 64 + l] = m[g][n] (0 past N), the scale layout of k_pack
__global__ void k_pack_scales(const int16_t* __restrict__ m, int16_t* __restrict__ mp, int N, int G, int64_t n,
                              int nb_off, int64_t nbs_tot) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(i & 63);
    const int64_t lt = i >> 6;
    const int g = (int)(lt % G);
    const int64_t nb = lt / G;
    const int64_t col = nb * 64 + l;
    mp[tile_index(nb + nb_off, g, nbs_tot, G) * 64 + l] = col < N ? m[(int64_t)g * N + col] : (int16_t)0;
  }
}

// emb[v][k] = rint(W[v][k] * M[k/128][v] / 4096), round half to even
__global__ void k_embed_table(const int8_t* __restrict__ wp, const int16_t* __restrict__ mp, int32_t* __restrict__ emb,
                              int V, int D, int G) {
  const int64_t total = (int64_t)V * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = i / D;
    const int k = (int)(i - v * D);
    const int64_t nb = v >> 6;
    const int l = (int)(v & 63), g = k >> 7, j = (k >> 4) & 7, b = k & 15;
    const int64_t tile = tile_index(nb, g, (V + 63) / 64, G);
    const int64_t a = (int64_t)wp[(tile * 8 + j) * 1024 + l * 16 + b] * (int64_t)mp[tile * 64 + l];
    int64_t q = a >> 12;
    const int64_t rem = a & 4095;
    if (rem > 2048 || (rem == 2048 && (q & 1))) q += 1;
    emb[i] = (int32_t)q;
  }
}

static int grid_for(int64_t n, int block = 256, int64_t cap = 1 << 16) {
  int64_t b = cdiv(n, block);
  if (b < 1) b = 1;
  return (int)(b > cap ? cap : b);
}

}  // namespace exact

using namespace exact;

static int check_part(int N, int K, int n_off, int Ntot) {
  if (N <= 0 || K <= 0 || n_off < 0 || Ntot < n_off + N) return EXACT_E_ARG;
  if (K % 128 || n_off % 64) return EXACT_E_UNSUPPORTED;
  return EXACT_OK;
}

extern "C" int exact_synth_linear(uint64_t key_w, uint64_t key_m, int32_t m_lo, int32_t m_hi, const uint32_t* thr,
                                  int8_t* wp, int16_t* mp, int32_t N, int32_t K, int32_t n_off, int32_t Ntot, void* stream) {
  if (!thr || !wp || !mp || m_hi <= m_lo || m_lo < 0 || m_hi > 32768) return EXACT_E_ARG;
  int e = check_part(N, K, n_off, Ntot);
  if (e) return e;
  if (reinterpret_cast<uintptr_t>(wp) & 15) return EXACT_E_UNSUPPORTED;
  hipStream_t st = as_stream(stream);
  const int G = K / 128;
  const int64_t nbs = cdiv(N, 64), nbs_tot = cdiv(Ntot, 64);
  const int64_t nch = nbs * G * 512;
  hipLaunchKernelGGL(k_synth_w, dim3(grid_for(nch)), dim3(256), 0, st, key_w, thr, wp, N, K, G, nch, n_off / 64, nbs_tot);
  const int64_t nm = nbs * G * 64;
  hipLaunchKernelGGL(k_synth_m, dim3(grid_for(nm)), dim3(256), 0, st, key_m, m_lo, m_hi, mp, N, G, nm, n_off / 64, nbs_tot);
  return launch_status("synth_linear");
}

extern "C" int exact_synth_vector(uint64_t key, int64_t lo, int64_t hi, int64_t* out, int64_t n, void* stream) {
  if (!out || n < 0 || hi <= lo || (uint64_t)(hi - lo) > 0xFFFFFFFFULL) return EXACT_E_ARG;
  if (n == 0) return EXACT_OK;
  hipLaunchKernelGGL(k_synth_vec, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), key, lo, (uint64_t)(hi - lo), out, n);
  return launch_status("synth_vector");
}

extern "C" int exact_pack_linear(const int8_t* w_kn, const int16_t* m_gn, int8_t* wp, int16_t* mp, int32_t N, int32_t K,
                                 int32_t n_off, int32_t Ntot, void* stream) {
  if (!w_kn || !m_gn || !wp || !mp) return EXACT_E_ARG;
  int e = check_part(N, K, n_off, Ntot);
  if (e) return e;
  if (reinterpret_cast<uintptr_t>(wp) & 15) return EXACT_E_UNSUPPORTED;
  const int G = K / 128;
  const int64_t nch = cdiv(N, 64) * G * 512;
  hipLaunchKernelGGL(k_pack, dim3(grid_for(nch)), dim3(256), 0, as_stream(stream), w_kn, m_gn, wp, mp, N, K, G, nch,
                     n_off / 64, cdiv(Ntot, 64));
  return launch_status("pack_linear");
}

extern "C" int exact_pack_scales(const int16_t* m_gn, int16_t* mp, int32_t N, int32_t K, int32_t n_off, int32_t Ntot,
                                 void* stream) {
  if (!m_gn || !mp) return EXACT_E_ARG;
  int e = check_part(N, K, n_off, Ntot);
  if (e) return e;
  const int G = K / 128;
  const int64_t n = cdiv(N, 64) * G * 64;
  hipLaunchKernelGGL(k_pack_scales, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), m_gn, mp, N, G, n, n_off / 64,
                     cdiv(Ntot, 64));
  return launch_status("pack_scales");
}

extern "C" int exact_embed_table(const int8_t* wp, const int16_t* mp, int32_t* emb, int32_t V, int32_t D, void* stream) {
  if (!wp || !mp || !emb || V <= 0 || D <= 0) return EXACT_E_ARG;
  if (D % 128) return EXACT_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_embed_table, dim3(grid_for((int64_t)V * D)), dim3(256), 0, as_stream(stream), wp, mp, emb, V, D,
                     D / 128);
  return launch_status("embed_table");
}
