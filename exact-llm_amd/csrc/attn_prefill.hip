// Exact integer attention for prefill on the matrix cores (gfx950): R query rows of one sequence, at
// increasing positions pos[r], against the keys 0..pos[r] of its cache slot. Same result as k_attention
// (exact_llm.py:170-176; exact_torch.py:142-166):
//   sc = shr((qq . kq) * INV, 32 - sq - sk); p = isoftmax(sc) (Q20); out = shr(p . v, 20)
// in three kernels over workspaces:
//   k_attn_scores  q.k exactly from int8 digits on v_mfma_i32_32x32x32_i8. With x = 256 hi + lo + 128
//                  (hi = x >> 8, lo = (x & 255) - 128, both int8):
//                    q.k = 65536 HH + 256 (HL + LH) + LL + 128 (sum q + sum k) - 16384 hd,
//                  every digit product sum |.| < 2^22, so each is exact in int32. Scores go to int64 rows.
//   k_attn_softmax the integer softmax of each row, written as three balanced int8 digit planes of p
//                  (p = d0 + 256 d1 + 65536 d2, d0, d1 in [-128, 127], d2 in [0, 16]), zero past pos[r].
//   k_attn_pv      p.v from the p digits and balanced int8 digit planes of v (k_vdigits: as many digits as
//                  the largest |v| of the KV head needs, 4 or 8): each digit-pair product summed over
//                  the keys is exact in int32 when grouped by shift s = a + b, and
//                  p.v = sum_s C_s 256^s modulo 2^64, the int64 product of the reference.
// Head dimension 128 (the configurations' attention prefill).
#include "exact_common.h"
#include "abi_util.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

namespace exact {

int zero_bytes(void* dst, int64_t nbytes, hipStream_t st);

#define AP_HD 128

// int16 -> (hi, lo - 128) int8 digits of 16 values held in two 16-byte chunks
__device__ __forceinline__ void split_digits(v4i p0, v4i p1, v4i& hi, v4i& lo) {
  hi[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x07050301u);
  hi[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x07050301u);
  hi[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x07050301u);
  hi[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x07050301u);
  lo[0] = __builtin_amdgcn_perm(p0[1], p0[0], 0x06040200u) ^ 0x80808080;
  lo[1] = __builtin_amdgcn_perm(p0[3], p0[2], 0x06040200u) ^ 0x80808080;
  lo[2] = __builtin_amdgcn_perm(p1[1], p1[0], 0x06040200u) ^ 0x80808080;
  lo[3] = __builtin_amdgcn_perm(p1[3], p1[2], 0x06040200u) ^ 0x80808080;
}

// sum of the 16 int16 values in two 16-byte chunks
__device__ __forceinline__ int sum16(v4i p0, v4i p1) {
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += (int)(int16_t)(p0[i] & 0xffff) + (int)(int16_t)(p0[i] >> 16);
    s += (int)(int16_t)(p1[i] & 0xffff) + (int)(int16_t)(p1[i] >> 16);
  }
  return s;
}

// Balanced base-256 digits of every v of the sequence, transposed: vdig[((kh * 8 + b) * hd + d) * kpad + j]
// for keys j < kpad (zeros from nkeys on); vbits[kh] = max bit length of |v| over the KV head (zeroed before).
// grid (kpad / 32, KV), block 256: 32 keys read row-major, staged in LDS, written 32 keys per (digit, dimension).
#define VD_STRIDE 36   // bytes per LDS row of 32 keys, padded against bank conflicts
__global__ __launch_bounds__(256) void k_vdigits(const int64_t* __restrict__ v, int sl, int KV, int Smax, int nkeys, int kpad,
                                                 int8_t* __restrict__ vdig, int32_t* __restrict__ vbits) {
  __shared__ __align__(16) int8_t st[8 * AP_HD * VD_STRIDE];
  const int kh = blockIdx.y, j0 = blockIdx.x * 32, tid = threadIdx.x;
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  int bl = 0;
#pragma unroll 4
  for (int i = 0; i < 32 * AP_HD / 256; ++i) {
    const int e = tid + 256 * i, key = e / AP_HD, d = e % AP_HD;
    int64_t x = j0 + key < nkeys ? v[(cbase + j0 + key) * AP_HD + d] : 0;
    const int b0 = bitlen64(abs64(x));
    bl = b0 > bl ? b0 : bl;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int64_t dg = ((x + 128) & 255) - 128;
      st[(b * AP_HD + d) * VD_STRIDE + key] = (int8_t)dg;
      x = (x - dg) >> 8;
    }
  }
  bl = wave_max_i32(bl);
  if ((tid & 63) == 0) atomicMax(vbits + kh, bl);
  __syncthreads();
  int8_t* dst = vdig + (int64_t)kh * 8 * AP_HD * kpad + j0;
#pragma unroll 4
  for (int i = 0; i < 8 * AP_HD * 8 / 256; ++i) {
    const int idx = tid + 256 * i, row = idx >> 3, w = idx & 7;   // row = b * hd + d, w = dword of 32 keys
    *reinterpret_cast<int32_t*>(dst + (int64_t)row * kpad + 4 * w) = *reinterpret_cast<const int32_t*>(st + row * VD_STRIDE + 4 * w);
  }
}

// grid (ceil(R / 32), H), one wave: 32 query rows of head h against key tiles of 32.
__global__ __launch_bounds__(64) void k_attn_scores(const int16_t* __restrict__ qq, const int32_t* __restrict__ sq,
                                                    const int16_t* __restrict__ kq, const int32_t* __restrict__ sk,
                                                    const int32_t* __restrict__ pos, int sl, int64_t* __restrict__ scores,
                                                    int R, int H, int KV, int Smax, int nkeys, int kpad, int INV) {
  __shared__ int sSq[32], sSh[32];
  const int h = blockIdx.y, q0 = blockIdx.x * 32, lane = threadIdx.x, l32 = lane & 31, half = lane >> 5;
  const int kh = h / (H / KV);
  const int qr = q0 + l32 < R ? q0 + l32 : R - 1;
  // query digits (A operand: row = query l32, k = 16 half + [0, 16) of each 32-wide block)
  v4i qh[4], ql[4];
  int sqs = 0;
  const v4i* qp = reinterpret_cast<const v4i*>(qq + ((int64_t)qr * H + h) * AP_HD);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const v4i a0 = qp[(32 * kb + 16 * half) / 8], a1 = qp[(32 * kb + 16 * half) / 8 + 1];
    split_digits(a0, a1, qh[kb], ql[kb]);
    sqs += sum16(a0, a1);
  }
  sqs += __shfl_xor(sqs, 32, 64);
  if (half == 0) {
    sSq[l32] = sqs;
    sSh[l32] = sq[(int64_t)qr * H + h];
  }
  __syncthreads();
  int rSq[16], rSh[16], rPos[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 8 * (i >> 2) + 4 * half + (i & 3);
    rSq[i] = sSq[row];
    rSh[i] = sSh[row];
    rPos[i] = q0 + row < R ? pos[q0 + row] : -1;
  }
  const int qlast = q0 + 31 < R ? q0 + 31 : R - 1;
  const int jmax = min(pos[qlast], nkeys - 1);   // positions increase with the row; never past the written keys
  const int64_t cbase = ((int64_t)sl * KV + kh) * Smax;
  for (int j0 = 0; j0 <= jmax; j0 += 32) {
    const int key = j0 + l32 <= jmax ? j0 + l32 : jmax;
    const v4i* kp = reinterpret_cast<const v4i*>(kq + (cbase + key) * AP_HD);
    v4i kh_[4], kl_[4];
    int sks = 0;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const v4i b0 = kp[(32 * kb + 16 * half) / 8], b1 = kp[(32 * kb + 16 * half) / 8 + 1];
      split_digits(b0, b1, kh_[kb], kl_[kb]);
      sks += sum16(b0, b1);
    }
    sks += __shfl_xor(sks, 32, 64);
    const int skv = sk[cbase + key];
    v16i hh = {}, x = {}, ll = {};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      hh = __builtin_amdgcn_mfma_i32_32x32x32_i8(qh[kb], kh_[kb], hh, 0, 0, 0);
      x = __builtin_amdgcn_mfma_i32_32x32x32_i8(qh[kb], kl_[kb], x, 0, 0, 0);
      x = __builtin_amdgcn_mfma_i32_32x32x32_i8(ql[kb], kh_[kb], x, 0, 0, 0);
      ll = __builtin_amdgcn_mfma_i32_32x32x32_i8(ql[kb], kl_[kb], ll, 0, 0, 0);
    }
    // C layout: lane holds key column l32 and query rows 8 (i / 4) + 4 half + i % 4
    const int col = j0 + l32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 8 * (i >> 2) + 4 * half + (i & 3);
      const int64_t dot = ((int64_t)hh[i] << 16) + ((int64_t)x[i] << 8) + (int64_t)ll[i] +
                          128 * (int64_t)(rSq[i] + sks) - 16384LL * AP_HD;
      if (col <= rPos[i] && col <= jmax) scores[((int64_t)h * R + q0 + row) * kpad + col] = shr64(dot * INV, 32 - rSh[i] - skv);
    }
  }
}

// grid (R, H), block 256: softmax of one score row -> three balanced digit planes of p (Q20), zero past pos
__global__ __launch_bounds__(256) void k_attn_softmax(const int64_t* __restrict__ scores, const int32_t* __restrict__ pos,
                                                      const int32_t* __restrict__ T, int8_t* __restrict__ pd, int R, int H,
                                                      int nkeys, int kpad) {
  __shared__ int64_t red_a[16], red_b[16];
  const int r = blockIdx.x, h = blockIdx.y;
  const int S = max(1, min(pos[r] + 1, nkeys));
  const int64_t* row = scores + ((int64_t)h * R + r) * kpad;
  int64_t mx = INT64_MIN;
  for (int j = threadIdx.x; j < S; j += blockDim.x) mx = row[j] > mx ? row[j] : mx;
  mx = block_max64(mx, red_a);
  int64_t es = 0;
  for (int j = threadIdx.x; j < S; j += blockDim.x) es += lut_exp(T, mx - row[j]);
  es = block_sum64(es, red_b);
  const int64_t plane = (int64_t)H * R * kpad;
  int8_t* out = pd + ((int64_t)h * R + r) * kpad;
  for (int j = threadIdx.x; j < kpad; j += blockDim.x) {
    int64_t p = j < S ? floordiv_pos(shl64(lut_exp(T, mx - row[j]), 20), es) : 0;
    const int64_t d0 = ((p + 128) & 255) - 128;
    p = (p - d0) >> 8;
    const int64_t d1 = ((p + 128) & 255) - 128;
    p = (p - d1) >> 8;
    out[j] = (int8_t)d0;
    out[plane + j] = (int8_t)d1;
    out[2 * plane + j] = (int8_t)p;
  }
}

// grid (ceil(R / 32), H), block 256: wave w owns dimensions [32 w, 32 w + 32) of 32 query rows.
template <int NB>
__device__ __forceinline__ void pv_tiles(const int8_t* __restrict__ pd, const int8_t* __restrict__ vd, int64_t plane,
                                         int64_t prow, int64_t vrow, int64_t vplane, int jmax, int half, v16i (&acc)[NB + 2]) {
#pragma unroll
  for (int s = 0; s < NB + 2; ++s) acc[s] = v16i{};
  for (int j0 = 0; j0 <= jmax; j0 += 32) {
    const int k0 = j0 + 16 * half;
    v4i pa[3], vb[NB];
#pragma unroll
    for (int a = 0; a < 3; ++a) pa[a] = *reinterpret_cast<const v4i*>(pd + a * plane + prow + k0);
#pragma unroll
    for (int b = 0; b < NB; ++b) vb[b] = *reinterpret_cast<const v4i*>(vd + b * vplane + vrow + k0);
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[a + b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa[a], vb[b], acc[a + b], 0, 0, 0);
  }
}

template <int NB>
__device__ __forceinline__ void pv_store(const v16i (&acc)[NB + 2], int64_t* __restrict__ out, int* rowbits, int q0, int R,
                                         int H, int h, int d, int half) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint64_t tot = 0;
#pragma unroll
    for (int s = 0; s < NB + 2; ++s) tot += (uint64_t)shl64((int64_t)acc[s][i], 8 * s);
    const int row = 8 * (i >> 2) + 4 * half + (i & 3);
    const int64_t o = shr64((int64_t)tot, 20);
    if (q0 + row < R) out[((int64_t)(q0 + row) * H + h) * AP_HD + d] = o;
    atomicMax(rowbits + row, bitlen64(abs64(o)));
  }
}

__global__ __launch_bounds__(256) void k_attn_pv(const int8_t* __restrict__ pd, const int8_t* __restrict__ vdig,
                                                 const int32_t* __restrict__ vbits, const int32_t* __restrict__ pos,
                                                 int64_t* __restrict__ out, int32_t* __restrict__ obits, int R, int H, int KV,
                                                 int nkeys, int kpad) {
  __shared__ int rowbits[32];
  const int h = blockIdx.y, q0 = blockIdx.x * 32, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, half = lane >> 5;
  const int kh = h / (H / KV);
  if (tid < 32) rowbits[tid] = 0;
  __syncthreads();
  const int qr = q0 + l32 < R ? q0 + l32 : R - 1;
  const int qlast = q0 + 31 < R ? q0 + 31 : R - 1;
  const int jmax = min(pos[qlast], nkeys - 1);
  const int64_t plane = (int64_t)H * R * kpad;
  const int64_t prow = ((int64_t)h * R + qr) * kpad;     // A: query row l32, keys k0 + [0, 16)
  const int d = 32 * w + l32;
  const int64_t vplane = (int64_t)AP_HD * kpad;
  const int64_t vrow = (int64_t)d * kpad;                 // B: dimension l32 of the wave's 32, keys k0 + [0, 16)
  const int8_t* vd = vdig + (int64_t)kh * 8 * vplane;
  const int nbits = vbits[kh];
  if (nbits + 2 <= 32) {   // |v| < 2^30: four balanced digits
    v16i acc[6];
    pv_tiles<4>(pd, vd, plane, prow, vrow, vplane, jmax, half, acc);
    pv_store<4>(acc, out, rowbits, q0, R, H, h, d, half);
  } else {
    v16i acc[10];
    pv_tiles<8>(pd, vd, plane, prow, vrow, vplane, jmax, half, acc);
    pv_store<8>(acc, out, rowbits, q0, R, H, h, d, half);
  }
  __syncthreads();
  if (obits && tid < 32 && q0 + tid < R) obits[(int64_t)(q0 + tid) * H + h] = rowbits[tid];
}

}  // namespace exact

using namespace exact;

extern "C" int exact_attention_prefill(const int16_t* qq, const int32_t* sq, const int16_t* kq, const int32_t* sk,
                                       const int64_t* v, int32_t slot, const int32_t* pos, const int32_t* exp_t, int64_t* out,
                                       int32_t* obits, int64_t* scores, int8_t* pdig, int8_t* vdig, int32_t* vbits,
                                       int32_t R, int32_t H, int32_t KV, int32_t hd, int32_t Smax, int32_t nkeys,
                                       int32_t INV, void* stream) {
  if (!qq || !sq || !kq || !sk || !v || !pos || !exp_t || !out || !scores || !pdig || !vdig || !vbits) return EXACT_E_ARG;
  if (R <= 0 || H <= 0 || KV <= 0 || H % KV || slot < 0 || Smax <= 0 || nkeys <= 0 || nkeys > Smax) return EXACT_E_ARG;
  // per shift class, 3 digit pairs x nkeys products of |.| <= 2^14 stay below 2^31
  if (hd != AP_HD || nkeys > 32768) return EXACT_E_UNSUPPORTED;
  const int kpad = (nkeys + 31) / 32 * 32;
  hipStream_t st = as_stream(stream);
  int e = zero_bytes(vbits, (int64_t)KV * 4, st);
  if (e) return e;
  hipLaunchKernelGGL(k_vdigits, dim3(kpad / 32, KV), dim3(256), 0, st, v, slot, KV, Smax, nkeys, kpad, vdig, vbits);
  hipLaunchKernelGGL(k_attn_scores, dim3((R + 31) / 32, H), dim3(64), 0, st, qq, sq, kq, sk, pos, slot, scores, R, H, KV, Smax,
                     nkeys, kpad, INV);
  hipLaunchKernelGGL(k_attn_softmax, dim3(R, H), dim3(256), 0, st, scores, pos, exp_t, pdig, R, H, nkeys, kpad);
  hipLaunchKernelGGL(k_attn_pv, dim3((R + 31) / 32, H), dim3(256), 0, st, pdig, vdig, vbits, pos, out, obits, R, H, KV, nkeys,
                     kpad);
  return launch_status("attention_prefill");
}
