"""exact_logits_argmax_noalloc (the entry point that allocates nothing) against exact_logits_argmax with a caller
workspace, both called through the C ABI: two calls in a row, the second on a smaller input, bit-exact logits,
greedy ids and cleared totals; sizes beyond the library-owned scratch are rejected with no launch."""
import ctypes

import numpy as np
import pytest
import torch

from exact_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(rng, R, N, lo, hi):
    t = torch.from_numpy(rng.integers(lo, hi, (R, N))).to(DEV)
    s = torch.from_numpy(rng.integers(0, 14, R).astype(np.int32)).to(DEV)
    # ties: the row maximum repeated further on, so the first index must win
    j = int(rng.integers(0, N // 2))
    t[:, N - 1 - j] = t.max(1).values + 4096
    t[:, j] = t[:, N - 1 - j]
    return t, s


def _run(fn, t, s, clear):
    R, N = t.shape
    tt = t.clone()
    lg = torch.empty_like(t)
    ids = torch.full((R,), -1, dtype=torch.int32, device=DEV)
    lib = _lib.load()
    if fn == "exact_logits_argmax":
        part = torch.empty(R * -(-N // 4096) * 2, dtype=torch.int64, device=DEV)
        rc = lib.exact_logits_argmax(_p(tt), _p(s), _p(lg), _p(ids), _p(part), R, N, int(clear), _stream())
    else:
        rc = lib.exact_logits_argmax_noalloc(_p(tt), _p(s), _p(lg), _p(ids), R, N, int(clear), _stream())
    assert rc == 0, (fn, rc, lib.exact_last_error())
    torch.cuda.synchronize()
    return tt.cpu().numpy(), lg.cpu().numpy(), ids.cpu().numpy()


@pytest.mark.parametrize("clear", [0, 1])
def test_noalloc_matches_workspace_entry_point(clear):
    rng = np.random.default_rng(41 + clear)
    for R, N in ((8, 152064), (3, 5000)):            # the second call is smaller: nothing stale may be read
        print(f"logits_argmax_noalloc R={R} N={N} clear={clear}", flush=True)
        t, s = _case(rng, R, N, -(1 << 44), 1 << 44)
        want = _run("exact_logits_argmax", t, s, clear)
        got = _run("exact_logits_argmax_noalloc", t, s, clear)
        for a, b in zip(want, got):
            assert np.array_equal(a, b), (R, N)
        assert np.array_equal(got[2], got[1].argmax(1))
        if clear:
            assert not got[0].any()


def test_noalloc_rejects_sizes_beyond_its_scratch():
    lib = _lib.load()
    t = torch.zeros((65, 64), dtype=torch.int64, device=DEV)
    s = torch.zeros(65, dtype=torch.int32, device=DEV)
    ids = torch.zeros(65, dtype=torch.int32, device=DEV)
    assert lib.exact_logits_argmax_noalloc(_p(t), _p(s), None, _p(ids), 65, 64, 0, _stream()) == 2      # R > 64
    assert lib.exact_logits_argmax_noalloc(_p(t), _p(s), None, _p(ids), 1, (1 << 20) + 1, 0, _stream()) == 2  # N > 2^20
