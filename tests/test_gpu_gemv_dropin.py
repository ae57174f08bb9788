"""exact::gemv as a drop-in for the reference's op: the reference's own tensors (x16 int16 (K,), wT int8 (N, K)
row-major, Mg int64 (N, K/128)) in, int64 (N,) out, no repacking.

test_reference_g1 is the reference's pre-registered G1 test (experiments/speed_fair_kaggle.py:703-711): the same six
layer shapes, inputs drawn in the same order from torch.Generator().manual_seed(0), and the same int64 closed form
((x_g * w_g).sum * Mg).sum computed on the CPU."""
import numpy as np
import pytest
import torch

import exact_oracle as O
from exact_amd import ops
from exact_amd._lib import ExactError

pytestmark = pytest.mark.gpu
DEV = "cuda"
E = torch.ops.exact


def test_reference_g1():
    g = torch.Generator().manual_seed(0)
    for K, N in ((896, 896), (896, 4864), (4864, 896), (1536, 8960), (8960, 1536), (896, 151936)):
        print(f"G1 K={K} N={N}", flush=True)
        x = torch.randint(-32767, 32768, (K,), generator=g, dtype=torch.int64)
        w = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int64)
        Mg = torch.randint(1, 1 << 27, (N, K // 128), generator=g, dtype=torch.int64)
        ref = ((x.view(K // 128, 128, 1) * w.view(K // 128, 128, N)).sum(1) * Mg.T).sum(0)
        got = E.gemv(x.to(torch.int16).to(DEV), w.to(torch.int8).T.contiguous().to(DEV), Mg.to(DEV)).cpu()
        assert torch.equal(got, ref), (K, N)


def closed_form(x, wT, Mg):
    acc = O.group_acc(x[None].astype(np.int64), wT.T.astype(np.int64))[:, 0, :]    # (G, N) exact int32 group sums
    return (acc * Mg.T).sum(0)                                                      # int64, wrapping like the reference


@pytest.mark.parametrize("N,K", [(1, 128), (63, 256), (65, 384), (300, 1280), (4608, 3584), (1000, 18944),
                                 (18949, 3584), (2053, 8192), (9001, 1152), (3584, 18944), (2049, 4224)])
def test_ragged_shapes_and_wrapping_scales(N, K):
    """Shapes that give a wave 1, 2, 4 and 8 rows (the last row block ragged: 18949 = 8 * 2368 + 5), K ranges of 4 KiB
    and 2 KiB (K >= 8192), and ranges whose last chunk is partly or barely used (3584, 1152); rows of several ranges
    combine with 64-bit atomics (the 7B down shape 3584 x 18944: 10 ranges; 2049 x 4224: the second range 128 bytes)."""
    rng = np.random.default_rng(N * 7 + K)
    x = rng.integers(-32768, 32768, K).astype(np.int16)
    wT = rng.integers(-128, 128, (N, K)).astype(np.int8)
    Mg = rng.integers(1, 1 << 27, (N, K // 128))
    Mg[:, -1] = rng.integers(-(1 << 62), 1 << 62, N)                                 # products and sums wrap mod 2^64
    got = E.gemv(torch.from_numpy(x).to(DEV), torch.from_numpy(wT).to(DEV), torch.from_numpy(Mg).to(DEV))
    assert np.array_equal(got.cpu().numpy(), closed_form(x, wT, Mg)), (N, K)


def test_extreme_group_sums():
    """Every product at its extreme: x = -32768, w = -128 gives the largest group sum, 128 * 2^22 = 2^29."""
    N, K = 128, 512
    x = np.full(K, -32768, np.int16)
    wT = np.full((N, K), -128, np.int8)
    wT[1::2] = 127
    Mg = np.full((N, K // 128), (1 << 27) - 1, np.int64)
    got = E.gemv(torch.from_numpy(x).to(DEV), torch.from_numpy(wT).to(DEV), torch.from_numpy(Mg).to(DEV))
    assert np.array_equal(got.cpu().numpy(), closed_form(x, wT, Mg))


def test_graph_capture_replays_match_eager():
    """The op captured in a HIP graph (as GraphDecoder captures TLinG) gives the eager result on every replay,
    with eager work and synchronisations between replays and the input changed in place."""
    rng = np.random.default_rng(3)
    N, K = 4864, 896
    x = torch.from_numpy(rng.integers(-32767, 32768, K).astype(np.int16)).to(DEV)
    wT = torch.from_numpy(rng.integers(-127, 128, (N, K)).astype(np.int8)).to(DEV)
    Mg = torch.from_numpy(rng.integers(1, 1 << 27, (N, K // 128))).to(DEV)
    E.gemv(x, wT, Mg)                                   # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = E.gemv(x, wT, Mg)
    for rep in range(4):
        x.copy_(torch.from_numpy(rng.integers(-32767, 32768, K).astype(np.int16)).to(DEV))
        want = E.gemv(x, wT, Mg).clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep
        assert np.array_equal(want.cpu().numpy(), closed_form(x.cpu().numpy(), wT.cpu().numpy(), Mg.cpu().numpy()))


def test_rejects_what_the_reference_would_misread():
    x = torch.zeros(200, dtype=torch.int16, device=DEV)
    with pytest.raises(ExactError):
        E.gemv(x, torch.zeros((64, 200), dtype=torch.int8, device=DEV), torch.zeros((64, 1), dtype=torch.int64, device=DEV))
    x = torch.zeros(256, dtype=torch.int16, device=DEV)
    with pytest.raises(ExactError):      # packed-style int16 scales are not the reference's Mg
        E.gemv(x, torch.zeros((64, 256), dtype=torch.int8, device=DEV), torch.zeros((64, 2), dtype=torch.int16, device=DEV))
    with pytest.raises(ExactError):      # (K, N) weight instead of wT (N, K)
        ops.gemv_rows(x, torch.zeros((256, 64), dtype=torch.int8, device=DEV), torch.zeros((64, 2), dtype=torch.int64,
                                                                                          device=DEV))
