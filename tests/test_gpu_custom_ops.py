"""The boundary's torch custom ops on the GPU give the same integers as the wrappers they call, and leave their
inputs unchanged (the wrappers are oracle-pinned in the other GPU tests)."""
import numpy as np
import pytest
import torch

from exact_amd import ops, synth
from exact_amd.tables import exp_t, silu_t

pytestmark = pytest.mark.gpu
DEV = "cuda"
E = torch.ops.exact
rng = np.random.default_rng(77)


def dev(a, dt):
    return torch.tensor(np.ascontiguousarray(a), dtype=dt, device=DEV)


def same(a, b):
    torch.cuda.synchronize()
    return np.array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_custom_ops_match_wrappers():
    thr = dev(synth.thresholds().astype(np.int64), torch.int64).to(torch.int32)
    N, K = 700, 512
    wp, mp = ops.PackedLinear.alloc(N, K, DEV)
    ops.synth_linear(wp, mp, N, K, synth.key(5, "w"), synth.key(5, "m"), synth.M_LO, synth.M_HI, thr)
    lin = ops.PackedLinear(wp, mp, N, K)
    for R, abits in ((5, 15), (100, 15), (64, 7)):
        lim = (1 << abits) - 1
        x = dev(rng.integers(-lim, lim + 1, (R, K)), torch.int16 if abits == 15 else torch.int8)
        assert same(E.gemm_g128(x, abits, wp, mp, N), ops.linear_t(x, abits, lin))
    xr = dev(rng.integers(-(1 << 36), 1 << 36, (3, 896)), torch.int64)
    g = dev(rng.integers(1 << 15, 1 << 17, 896), torch.int64)
    x0 = xr.clone()
    xq, s = E.rmsnorm_qrow(xr, g, 15)
    wq, ws = ops.rmsnorm_qrow(xr.clone(), g, 15)
    assert same(xq, wq) and same(s, ws) and same(xr, x0)
    t = dev(rng.integers(-(1 << 44), 1 << 44, (2, 2 * 1408)), torch.int64)
    sh = dev(rng.integers(0, 8, 2), torch.int32)
    silu = dev(silu_t(), torch.int32)
    t0 = t.clone()
    hq, hs = E.swiglu_qrow(t, sh, silu, 15)
    wq, ws = ops.swiglu_qrow(t.clone(), sh, silu, 15)
    assert same(hq, wq) and same(hs, ws) and same(t, t0)
    expt = dev(exp_t(), torch.int32)
    H, KV, hd, Smax = 4, 2, 128, 40
    kq = dev(rng.integers(-32767, 32768, (2, KV, Smax, hd)), torch.int16)
    sk = dev(rng.integers(0, 4, (2, KV, Smax)), torch.int32)
    v = dev(rng.integers(-(1 << 29), 1 << 29, (2, KV, Smax, hd)), torch.int64)
    qq = dev(rng.integers(-32767, 32768, (2, H, hd)), torch.int16)
    sq = dev(rng.integers(0, 4, (2, H)), torch.int32)
    slot, pos = dev([1, 0], torch.int32), dev([30, 7], torch.int32)
    out = torch.empty((2, H * hd), dtype=torch.int64, device=DEV)
    assert same(E.attention(qq, sq, kq, sk, v, slot, pos, expt, 5793),
                ops.attention(qq, sq, (kq, sk, v), slot, pos, expt, out, H, KV, hd, 5793))
    tr = dev(rng.integers(-(1 << 40), 1 << 40, (4, 60)), torch.int64)
    s4 = dev(rng.integers(0, 8, 4), torch.int32)
    tr0 = tr.clone()
    p, e = E.router_topk(tr, s4, expt, 4)
    wp_, we_ = torch.empty((4, 4), dtype=torch.int64, device=DEV), torch.empty((4, 4), dtype=torch.int32, device=DEV)
    ops.router_topk(tr.clone(), s4, expt, 4, wp_, we_)
    assert same(p, wp_) and same(e, we_) and same(tr, tr0)
    th = dev(rng.integers(-(1 << 40), 1 << 40, (2, 5000)), torch.int64)
    lg, ids = E.logits_argmax(th, sh)
    assert same(ids.long(), lg.argmax(1))
    wl = ops.logits_argmax(th.clone(), sh, torch.empty_like(th), torch.empty(2, dtype=torch.int32, device=DEV))[0]
    assert same(lg, wl)
