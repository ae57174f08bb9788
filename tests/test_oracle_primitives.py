"""Brute-force and closed-form checks of the oracle's integer primitives (Python ints as ground truth)."""
import math

import numpy as np
import pytest

import exact_oracle as O

rng = np.random.default_rng(11)


def py_shr(a, n):
    return a << -n if n <= 0 else (a + (1 << (n - 1))) >> n


def test_round_shift_scalar_and_array():
    a = rng.integers(-(1 << 50), 1 << 50, 4000)
    for n in (-5, 0, 1, 2, 7, 16, 28, 40):
        got = O.round_shift(a, n)
        assert [int(v) for v in got] == [py_shr(int(v), n) for v in a]
    n = rng.integers(-8, 40, 4000)
    got = O.round_shift(a, n)
    assert [int(v) for v in got] == [py_shr(int(x), int(k)) for x, k in zip(a, n)]
    # half-up on ties, negative values included
    assert list(O.round_shift(np.array([1, 3, -1, -3, 2, -2]), 1)) == [1, 2, 0, -1, 1, -1]


def test_bitlen_matches_int_bit_length():
    v = np.concatenate([rng.integers(0, 1 << 62, 3000), np.array([0, 1, 2, 3, (1 << 32) - 1, 1 << 32, (1 << 53) + 1,
                                                                  (1 << 63) - 1], np.int64)])
    for sh in (0, 5, 20, 33, 45):
        w = v >> sh
        assert [int(b) for b in O.bitlen(w)] == [int(x).bit_length() for x in w]
    assert list(O.bitlen(np.array([-5, 0]))) == [0, 0]


def test_qrow_brute_force():
    for bits in (7, 15):
        x = rng.integers(-(1 << 40), 1 << 40, (9, 300)) >> rng.integers(0, 40, (9, 1))
        xq, s = O.qrow(x, bits)
        lim = (1 << bits) - 1
        for r in range(x.shape[0]):
            m = max(abs(int(v)) for v in x[r])
            sr = max(m.bit_length() - bits, 0)
            assert int(s[r, 0]) == sr
            assert [int(v) for v in xq[r]] == [max(-lim, min(lim, py_shr(int(v), sr))) for v in x[r]]
            assert np.abs(xq[r]).max() <= lim


def test_isqrt_exact():
    n = np.concatenate([rng.integers(0, 1 << 62, 5000), np.arange(0, 2000),
                        np.array([k * k for k in rng.integers(1, 1 << 31, 500)] +
                                 [k * k - 1 for k in rng.integers(1, 1 << 31, 500)], np.int64)])
    assert [int(r) for r in O.isqrt(n)] == [math.isqrt(int(v)) for v in n]


def py_irms(x, g):
    m = max(abs(v) for v in x)
    k = max(m.bit_length() - 24, 0)
    xs = [py_shr(v, k) for v in x]
    ms = sum(v * v for v in xs) // len(x) + 1
    r = max(math.isqrt(ms), 1)
    return [py_shr(((v << 16) // (r << k)) * gi, 16) for v, gi in zip(x, g)]


def test_irms_brute_force_negative_floor_division():
    for scale in (10, 20, 30, 40):
        x = rng.integers(-(1 << scale), 1 << scale, (3, 256))
        g = rng.integers(1 << 15, 1 << 17, 256)
        got = O.irms(x, g)
        for r in range(3):
            assert [int(v) for v in got[r]] == py_irms([int(v) for v in x[r]], [int(v) for v in g])


def py_isoftmax(sc, valid, T):
    mx = max(s for s, ok in zip(sc, valid) if ok)
    es = []
    for s, ok in zip(sc, valid):
        d = mx - s if ok else 0
        i = min(d >> 8, len(T) - 2)
        fr = d & 255
        e = int(T[i]) - py_shr((int(T[i]) - int(T[i + 1])) * fr, 8)
        es.append(e if ok and d < (40 << 16) else 0)
    tot = sum(es)
    return [(e << 20) // tot for e in es]


def test_isoftmax_brute_force():
    sc = rng.integers(-(1 << 22), 1 << 22, (6, 50))
    valid = rng.random((6, 50)) < 0.7
    valid[:, 0] = True
    p = O.isoftmax(sc, valid)
    for r in range(6):
        assert [int(v) for v in p[r]] == py_isoftmax([int(v) for v in sc[r]], list(valid[r]), O.EXP_T)
    assert (p[~valid] == 0).all()
    assert (p.sum(-1) <= 1 << 20).all() and (p.sum(-1) > (1 << 20) - 50).all()


def test_lut_nonlinearities_closed_form():
    x = np.concatenate([rng.integers(-(20 << 16), 20 << 16, 4000),
                        np.array([-(16 << 16) - 1, -(16 << 16), (16 << 16) - 1, 16 << 16, 0])])
    y = O.isilu(x)
    s = O.isig(x)
    for v, a, b in zip(x, y, s):
        v = int(v)
        if v >= 16 << 16:
            assert int(a) == v and int(b) == 1 << 16
        elif v < -(16 << 16):
            assert int(a) == 0 and int(b) == 0
        else:
            t = v + (16 << 16)
            i, fr = t >> 8, t & 255
            assert int(a) == int(O.SILU_T[i]) + py_shr((int(O.SILU_T[i + 1]) - int(O.SILU_T[i])) * fr, 8)
            assert int(b) == int(O.SIG_T[i]) + py_shr((int(O.SIG_T[i + 1]) - int(O.SIG_T[i])) * fr, 8)
    # tables against their mathematics (within rounding of the Q16 / Q24 value)
    v = (np.arange(len(O.SIG_T)) - 4096) / 256
    assert np.abs(O.SIG_T - 65536 / (1 + np.exp(-v))).max() <= 0.5 + 1e-6
    assert np.abs(O.SILU_T - 65536 * v / (1 + np.exp(-v))).max() <= 0.5 + 1e-6
    assert O.SIG_T[4096] == 32768 and O.SILU_T[4096] == 0


def test_group_linear_closed_form_g1():
    """speed_fair_kaggle.py:704-710: out = ((x*w) summed per group * Mg^T).sum(0), int64 brute force."""
    for K, N in ((896, 96), (256, 130), (1408, 64)):
        x = rng.integers(-32767, 32768, K)
        w = rng.integers(-127, 128, (K, N)).astype(np.int8)
        Mg = rng.integers(1, 1 << 27, (K // 128, N))
        ref = ((x.reshape(K // 128, 128, 1) * w.astype(np.int64).reshape(K // 128, 128, N)).sum(1) * Mg).sum(0)
        acc = O.group_acc(x[None, :], w)
        assert np.array_equal((acc[:, 0, :] * Mg).sum(0), ref)
        # full linear: y = shr(t, 28 - s) with s from qrow(x, 15) (here x already fits, s = 0)
        y, t = O.linear_group_t(x[None, :], w, Mg)
        assert np.array_equal(t[0], ref) and np.array_equal(y[0], O.round_shift(ref, 28))


def test_group_linear_abits_and_bias():
    x = rng.integers(-(1 << 30), 1 << 30, (5, 384))
    w = rng.integers(-127, 128, (384, 70)).astype(np.int8)
    Mg = rng.integers(1, 1 << 15, (3, 70))
    b = rng.integers(-1000, 1000, 70)
    for bits in (7, 15):
        xq, s = O.qrow(x, bits)
        t = np.zeros((5, 70), object)
        for r in range(5):
            for n in range(70):
                t[r, n] = sum(sum(int(xq[r, k]) * int(w[k, n]) for k in range(g * 128, g * 128 + 128)) * int(Mg[g, n])
                              for g in range(3))
        y = O.linear_group(x, w, Mg, b, abits=bits)
        exp = [[py_shr(int(t[r, n]), 28 - int(s[r, 0])) + int(b[n]) for n in range(70)] for r in range(5)]
        assert y.tolist() == exp


def test_channel_drop_rule():
    acc = np.array([[1 << 40, -(1 << 39), 5]], np.int64)
    M = np.array([1 << 26, 3, 7], np.int64)
    Mbits = 27
    s = np.array([[2]])
    drop = max((1 << 40).bit_length() + Mbits - 62, 0)
    assert drop == 6
    y = O.requant_channel(acc, s, M, Mbits)
    exp = [py_shr(py_shr(int(a), drop) * int(m), 28 - 2 - drop) for a, m in zip(acc[0], M)]
    assert y[0].tolist() == exp
    # no drop when the bound allows it
    small = np.array([[1000, -7, 3]], np.int64)
    assert O.requant_channel(small, s, M, Mbits)[0].tolist() == [py_shr(int(a) * int(m), 26) for a, m in zip(small[0], M)]


def test_splitmix64_known_answers():
    """SplitMix64 seeded with 0 (Steele, Lea, Flood 2014): first outputs of the published generator."""
    assert O.splitmix64(0, 0) == 0xE220A8397B1DCDAF
    assert O.splitmix64(0, 1) == 0x6E789E6AA1B965F4
    assert O.splitmix64(0, 2) == 0x06C45D188009454F


def test_sample_int_inverse_cdf_brute_force():
    lg = rng.integers(-(8 << 16), 8 << 16, 300)
    tnum = O.temp_num(0.8)
    for seed in range(5):
        tok, p = O.sample_int(lg, seed, 3, tnum)
        target = (O.u20(seed, 3) * int(p.sum())) >> 20
        c = 0
        for i, v in enumerate(p):
            c += int(v)
            if c > target:
                assert tok == i
                break


def test_rope_tables_and_rotation():
    cos, sin = O.rope_tables(40, 16, 1e4)
    assert cos[0].tolist() == [65536] * 16 and sin[0].tolist() == [0] * 16
    x = rng.integers(-(1 << 20), 1 << 20, (3, 40, 16))
    y = O.rope(x, cos, sin)
    t, i = 7, 3
    a, b = int(x[1, t, i]), int(x[1, t, i + 8])
    assert int(y[1, t, i]) == py_shr(a * int(cos[t, i]) - b * int(sin[t, i]), 16)
    assert int(y[1, t, i + 8]) == py_shr(b * int(cos[t, i + 8]) + a * int(sin[t, i + 8]), 16)


@pytest.mark.parametrize("hd,inv", [(16, 16384), (32, 11585), (64, 8192), (128, 5793)])
def test_inv_sqrt_hd(hd, inv):
    assert O.inv_sqrt_hd(hd) == inv
