/* C restatement of the two oracle routines that dominate large-model fixture runs.
 *
 * TEST INFRASTRUCTURE: this file belongs to the oracle. Only tests/, the fixture scripts under
 * tests/golden/ and the CPU-baseline leg of bench.py load it, and only as the reference results are compared
 * with. The product
 * never links or calls it.
 *
 *   oc_weights      the seeded int8 weight generator, the same law as exact_amd.synth.weights_np:
 *                   W[n][k] = -127 + #{j : thr[j] <= u}, with u = splitmix64(key, n*K + k) >> 32,
 *                   written in the oracle's (K, N) layout for rows [n0, n1)
 *   oc_scales       the group scales M[g][n] = lo + ((u * (hi - lo)) >> 32), u = splitmix64(key, n*G + g) >> 32
 *   oc_group_linear t[r][n] = sum_g M[g][n] * sum_{k in g} x[r][k] * w[k][n]      (GQLin,
 *                   experiments/speed_fair_kaggle.py:714-725; SPEC.md:18). Every group sum is exact in
 *                   int32 (|x| < 2^15, |w| <= 127, 128 terms), and t accumulates in int64.
 *
 * Pinned by tests/test_oracle_c.py against the numpy oracle (exact_oracle.linear_group_t and
 * exact_amd.synth.weights_np / scales_np) on random and edge-case inputs.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint64_t splitmix64(uint64_t key, uint64_t idx) {
  uint64_t z = key + (idx + 1ULL) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

void oc_weights(uint64_t key, const uint32_t* thr, int64_t N, int64_t K, int64_t n0, int64_t n1, int8_t* out) {
  const int64_t W = n1 - n0;
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < K; ++k) {
    int8_t* row = out + k * W;
    for (int64_t n = n0; n < n1; ++n) {
      const uint32_t u = (uint32_t)(splitmix64(key, (uint64_t)n * (uint64_t)K + (uint64_t)k) >> 32);
      int lo = 0, hi = 254;   /* first j with thr[j] > u */
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (thr[mid] <= u) lo = mid + 1; else hi = mid;
      }
      row[n - n0] = (int8_t)(lo - 127);
    }
  }
  (void)N;
}

void oc_scales(uint64_t key, int64_t lo, int64_t hi, int64_t N, int64_t G, int64_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < G; ++g)
    for (int64_t n = 0; n < N; ++n) {
      const uint64_t u = splitmix64(key, (uint64_t)n * (uint64_t)G + (uint64_t)g) >> 32;
      out[g * N + n] = lo + (int64_t)((u * (uint64_t)(hi - lo)) >> 32);
    }
}

/* x: (R, K) int16 (xbytes 2) or int8 (xbytes 1); w: (K, N) int8; M: (G, N) int64; t: (R, N) int64 */
void oc_group_linear(const void* x, int xbytes, int64_t R, int64_t K, const int8_t* w, int64_t N, const int64_t* M,
                     int64_t* t) {
  const int64_t G = K / 128;
  const int64_t CW = 2048;   /* columns per task */
  const int64_t ntask = (N + CW - 1) / CW;
#pragma omp parallel for schedule(dynamic)
  for (int64_t task = 0; task < ntask; ++task) {
    const int64_t c0 = task * CW, c1 = c0 + CW < N ? c0 + CW : N, cw = c1 - c0;
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(R * cw));
    int64_t* tot = (int64_t*)calloc((size_t)(R * cw), sizeof(int64_t));
    for (int64_t g = 0; g < G; ++g) {
      memset(acc, 0, sizeof(int32_t) * (size_t)(R * cw));
      for (int64_t k = g * 128; k < g * 128 + 128; ++k) {
        const int8_t* wr = w + k * N + c0;
        for (int64_t r = 0; r < R; ++r) {
          const int32_t xv = xbytes == 2 ? ((const int16_t*)x)[r * K + k] : ((const int8_t*)x)[r * K + k];
          if (!xv) continue;
          int32_t* ar = acc + r * cw;
          for (int64_t c = 0; c < cw; ++c) ar[c] += xv * (int32_t)wr[c];
        }
      }
      const int64_t* mg = M + g * N + c0;
      for (int64_t r = 0; r < R; ++r)
        for (int64_t c = 0; c < cw; ++c) tot[r * cw + c] += (int64_t)acc[r * cw + c] * mg[c];
    }
    for (int64_t r = 0; r < R; ++r) memcpy(t + r * N + c0, tot + r * cw, sizeof(int64_t) * (size_t)cw);
    free(acc);
    free(tot);
  }
}

/* Q16 embedding rows from the int8 table in the oracle's (K = D, N = V) layout:
 * emb[v][k] = rint(w[k][v] * M[k / 128][v] / 2^12), ties to even (numpy rint; exact_amd.synth.embed_np). */
void oc_embed(const int8_t* w, const int64_t* M, int64_t D, int64_t V, int64_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t v = 0; v < V; ++v)
    for (int64_t k = 0; k < D; ++k) {
      const int64_t a = (int64_t)w[k * V + v] * M[(k / 128) * V + v];
      int64_t q = a >> 12;
      const int64_t rem = a & 4095;
      if (rem > 2048 || (rem == 2048 && (q & 1))) q += 1;
      out[v * D + k] = q;
    }
}
