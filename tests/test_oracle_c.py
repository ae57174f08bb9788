"""The oracle's C restatement (oracle/exact_c.c) against the numpy oracle it accelerates."""
import numpy as np
import pytest

import exact_c
import exact_oracle as O
import helpers
from exact_amd import synth


@pytest.fixture(scope="module", autouse=True)
def lib():
    exact_c.load()
    yield
    exact_c.uninstall()


@pytest.mark.parametrize("N,K,n0,n1", [(64, 128, 0, 64), (300, 256, 0, 300), (1000, 384, 129, 700)])
def test_weights_and_scales_match_numpy_generator(N, K, n0, n1):
    k = synth.key(5, f"w{N}")
    assert np.array_equal(exact_c.weights(k, synth.thresholds(), N, K, n0, n1), synth.weights_np(k, N, K, n0, n1))
    assert np.array_equal(exact_c.scales(k, N, K, synth.M_LO, synth.M_HI), synth.scales_np(k, N, K))
    if K >= 128 and n0 == 0:
        w, M = synth.weights_np(k, N, K), synth.scales_np(k, N, K)
        M[0, :5] = [4096, 2048, 6144, 1, 8191]              # exact ties at .5 of both parities
        assert np.array_equal(exact_c.embed(w, M), synth.embed_np(w, M))


@pytest.mark.parametrize("R,K,N,lim", [(1, 128, 64, 32767), (5, 512, 3000, 32767), (37, 256, 130, 127), (3, 1024, 77, 0)])
def test_group_linear_matches_numpy(R, K, N, lim):
    rng = np.random.default_rng(R * K)
    x = rng.integers(-lim, lim + 1, (R, K)) if lim else np.zeros((R, K), np.int64)
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    M = rng.integers(1, 1 << 15, (K // 128, N))
    want = (O.group_acc(x, w) * M[:, None, :]).sum(0)
    assert np.array_equal(exact_c.group_t(x, w, M), want)


def test_group_linear_extremes():
    """Largest |group sum| (2^15-1) * 127 * 128 and largest scales, all signs."""
    K, N = 384, 130
    x = np.full((2, K), 32767)
    x[1, ::2] = -32767
    w = np.full((K, N), 127, np.int8)
    w[:, ::3] = -127
    M = np.full((K // 128, N), (1 << 15) - 1)
    want = (O.group_acc(x, w) * M[:, None, :]).sum(0)
    assert np.array_equal(exact_c.group_t(x, w, M), want)


def test_model_forward_identical_with_c_linear():
    cfg = synth.CONFIGS["tiny"]
    om = helpers.oracle_model(cfg, 2, T=32)
    ids = helpers.prompt(1, 9, cfg.V)
    exact_c.uninstall()
    want = om(ids)
    exact_c.install()
    try:
        assert np.array_equal(om(ids), want)
    finally:
        exact_c.uninstall()
