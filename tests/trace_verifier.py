"""Verifier side of the trace experiments, used by the tests to check captured traces (test infrastructure, not part
of the package): the Freivalds keys and check of gpu_engine_trace_verify_kaggle.py:799-833.

For a prime p and random r in [0, p)^N, the key of a linear is d = W'^T r mod p with W'[k][n] = W[k][n] * M[k // 128][n]
(group) or W (channel); a row of totals t passes when sum_n t[n] r[n] = sum_k xq[k] d[k] (mod p), for both primes.
"""
import numpy as np

P1, P2 = 2147483647, 2147483629   # the reference's two Freivalds primes (gpu_engine_trace_verify_kaggle.py:782)


def freivalds_keys(w, M=None, rng=None, primes=(P1, P2), chunk=2048):
    """Keys (p, r, d) of one linear for each prime p (gpu_engine_trace_verify_kaggle.py:799-815): w (K, N) int8,
    M (K/128, N) group scales or None (channel mode: t = xq . W). d = W'^T r mod p, every product reduced mod p
    before a sum of at most `chunk` terms (all below 2^63)."""
    rng = np.random.default_rng() if rng is None else rng
    w = np.asarray(w, np.int64)
    K, N = w.shape
    out = []
    for p in primes:
        r = rng.integers(0, p, N, dtype=np.int64)
        d = np.zeros(K, np.int64)
        for g0 in range(0, K, 128):
            Wg = w[g0:g0 + 128] if M is None else w[g0:g0 + 128] * np.asarray(M, np.int64)[g0 // 128][None, :]
            Wg = Wg % p
            for j in range(0, N, chunk):
                d[g0:g0 + 128] = (d[g0:g0 + 128] + ((Wg[:, j:j + chunk] * r[j:j + chunk][None, :]) % p).sum(1)) % p
        out.append((p, r, d))
    return out


def _dot_mod(a, v, p, chunk=2048):
    """(a . v) mod p per row for int64 a (R, n) and v (n,) in [0, p): products reduced mod p before summing."""
    a = np.asarray(a, np.int64) % p
    acc = np.zeros(a.shape[0], np.int64)
    for j in range(0, a.shape[1], chunk):
        acc = (acc + ((a[:, j:j + chunk] * v[j:j + chunk][None, :]) % p).sum(1)) % p
    return acc


def freivalds_check(keys, xq, t):
    """True when every row of totals t (R, N) is consistent with the quantised inputs xq (R, K) under all keys
    (gpu_engine_trace_verify_kaggle.py:816-820)."""
    t = np.atleast_2d(np.asarray(t, np.int64))
    xq = np.atleast_2d(np.asarray(xq, np.int64))
    if t.shape[1] != keys[0][1].shape[0] or xq.shape[1] != keys[0][2].shape[0] or t.shape[0] != xq.shape[0]:
        return False
    return all(bool((_dot_mod(t, r, p) == _dot_mod(xq, d, p)).all()) for p, r, d in keys)
