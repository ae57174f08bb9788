"""Host side of trace capture (experiments/prover_commit_cost_gpu_kaggle.py:791-845,
experiments/gpu_engine_trace_verify_kaggle.py:799-833): the commitment, the Freivalds keys and check, and
the trace layout. Everything here runs without a GPU."""
import hashlib
from types import SimpleNamespace

import numpy as np
import pytest

from exact_amd import trace as TR
import trace_verifier as TV
from exact_amd.ops import ExactError


def test_commit_is_sha256_over_four_leaf_digests():
    a = np.arange(-5, 1000, dtype=np.int64) * 1234567891011
    step = (len(a) + 3) // 4
    b = a.astype("<i8").tobytes()
    leaves = [hashlib.sha256(b[8 * i * step:8 * (i + 1) * step]).digest() for i in range(4)]
    assert TR.commit(a) == hashlib.sha256(b"".join(leaves)).digest()
    a2 = a.copy()
    a2[777] += 1
    assert TR.commit(a2) != TR.commit(a)
    # a 1-element array: three empty leaves
    e = hashlib.sha256(b"").digest()
    one = np.array([7], np.int64)
    assert TR.commit(one) == hashlib.sha256(hashlib.sha256(one.tobytes()).digest() + e * 3).digest()


def _exact_t(xq, w, M):
    """t = sum_g M_g (xq_g . w_g) with Python integers."""
    R, K = xq.shape
    N = w.shape[1]
    t = np.zeros((R, N), dtype=object)
    for r in range(R):
        for n in range(N):
            t[r, n] = sum(int(M[g, n]) * sum(int(xq[r, k]) * int(w[k, n]) for k in range(128 * g, 128 * g + 128))
                          for g in range(K // 128))
    return t


def test_freivalds_keys_are_w_prime_times_r_mod_p():
    rng = np.random.default_rng(5)
    K, N = 256, 40
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    M = rng.integers(1, 1 << 15, (K // 128, N))
    keys = TV.freivalds_keys(w, M, np.random.default_rng(1), chunk=16)
    for p, r, d in keys:
        for k in (0, 1, 127, 128, 255):
            want = sum(int(w[k, n]) * int(M[k // 128, n]) * int(r[n]) for n in range(N)) % p
            assert int(d[k]) == want
    ck = TV.freivalds_keys(w, None, np.random.default_rng(1))
    for p, r, d in ck:
        assert int(d[3]) == sum(int(w[3, n]) * int(r[n]) for n in range(N)) % p


def test_freivalds_accepts_exact_totals_and_rejects_any_single_change():
    rng = np.random.default_rng(6)
    K, N, R = 256, 24, 3
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    M = rng.integers(8192, 24576, (K // 128, N))
    xq = rng.integers(-32767, 32768, (R, K))
    t = _exact_t(xq, w, M).astype(np.int64)
    keys = TV.freivalds_keys(w, M, np.random.default_rng(2))
    assert TV.freivalds_check(keys, xq, t)
    for i in range(20):
        bad = t.copy()
        bad[rng.integers(R), rng.integers(N)] += 1 if i % 2 else -1
        assert not TV.freivalds_check(keys, xq, bad)
    bx = xq.copy()
    bx[1, 200] += 1
    assert not TV.freivalds_check(keys, bx, t)
    assert not TV.freivalds_check(keys, xq, t[:, :-1])


def test_layout_offsets_and_reference_names():
    lin = lambda N, parts: SimpleNamespace(N=N, parts=parts)
    L = dict(qkv=lin(192, [("q", 0, 128), ("k", 128, 32), ("v", 160, 32)]), o=lin(128, [("o", 0, 128)]),
             gateup=lin(512, [("gate", 0, 256), ("up", 256, 256)]), down=lin(128, [("down", 0, 128)]))
    wts = SimpleNamespace(mode="group", cfg=SimpleNamespace(moe=False), layers=[L, L], head=lin(300, [("", 0, 300)]))
    R = 2
    lay = TR.TraceLayout(wts, R)
    per_layer = R * (192 + 128 + 512 + 128)
    assert lay.total == 2 * per_layer + R * 300
    buf = np.arange(lay.total, dtype=np.int64)
    parts = lay.split(buf)
    assert sorted(parts) == sorted([f"L{i}.{n}" for i in range(2) for n in ("q", "k", "v", "o", "gate", "up", "down")]
                                   + ["head"])
    assert parts["L0.q"].shape == (R, 128) and parts["L0.q"][1, 0] == 192
    assert parts["L0.v"][0, 0] == 160
    assert parts["L1.up"][0, 0] == per_layer + R * (192 + 128) + 256
    assert parts["head"][1, 299] == lay.total - 1
    with pytest.raises(ExactError):
        TR.TraceLayout(SimpleNamespace(mode="channel", cfg=SimpleNamespace(moe=False), layers=[], head=None), 1)
