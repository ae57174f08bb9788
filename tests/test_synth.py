"""The seeded integer artifact generator (host side): distribution, determinism, layout helpers."""
import math

import numpy as np

from exact_amd import synth


def test_thresholds_are_the_rounded_clipped_normal():
    thr = synth.thresholds().astype(np.float64) / 2 ** 32
    assert len(thr) == 254 and np.all(np.diff(thr) >= 0)
    # P(w = j) for the law of clip(rint(N(0, 40^2)), -127, 127)
    p = np.diff(np.concatenate([[0.0], thr, [1.0]]))
    j = np.arange(-127, 128)
    mean = float((p * j).sum())
    sd = math.sqrt(float((p * j * j).sum()) - mean ** 2)
    assert abs(mean) < 1e-6 and abs(sd - 39.9) < 0.2
    phi = lambda z: 0.5 * math.erfc(-z / math.sqrt(2))
    assert abs(p[127] - (phi(0.5 / 40) - phi(-0.5 / 40))) < 1e-9          # w = 0
    assert abs(p[0] - phi(-126.5 / 40)) < 1e-9                            # clipped tail at -127


def test_weights_empirical_law_and_determinism():
    k = synth.key(5, "x")
    w = synth.weights_np(k, 512, 1024)
    assert w.dtype == np.int8 and w.shape == (1024, 512)
    assert abs(float(w.mean())) < 0.3 and abs(float(w.std()) - 39.9) < 0.3
    assert np.array_equal(w, synth.weights_np(k, 512, 1024))
    assert np.array_equal(w[:, 100:200], synth.weights_np(k, 512, 1024, 100, 200))
    assert not np.array_equal(w, synth.weights_np(synth.key(6, "x"), 512, 1024))


def test_scales_and_vectors_in_range():
    M = synth.scales_np(synth.key(1, "m"), 300, 896)
    assert M.shape == (7, 300) and M.min() >= synth.M_LO and M.max() < synth.M_HI
    v = synth.vector_np(synth.key(1, "g"), 1000, *synth.GAIN)
    assert v.min() >= synth.GAIN[0] and v.max() < synth.GAIN[1]


def test_splitmix_matches_scalar_definition():
    k = synth.key(3, "t")
    idx = np.array([0, 1, 2, 12345, 2 ** 40], np.uint64)
    mask = (1 << 64) - 1

    def sm(key, i):
        z = (key + (i + 1) * 0x9E3779B97F4A7C15) & mask
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)
    assert [int(v) for v in synth.splitmix64_np(k, idx)] == [sm(k, int(i)) for i in idx]


def test_embed_rows_round_half_even():
    E = np.array([[1, -1, 3, 2]], np.int8).repeat(128, 0)          # (K=128, N=4)
    M = np.array([[2048, 2048, 2048, 6144]], np.int64)            # products 2048, -2048, 6144, 12288
    rows = synth.embed_np(E, M)
    assert rows[:, 0].tolist() == [0, 0, 2, 3]                      # rint(0.5)=0, rint(-0.5)=0, rint(1.5)=2, 3


def test_param_bytes_7b():
    b = synth.param_bytes(synth.CONFIGS["qwen2.5-7b"])
    assert abs(b - 7.18e9) / 7.18e9 < 0.01
