"""The boundary under torch.compile and HIP-graph capture, as the reference uses it.

The reference compiles its decode step, which calls its custom op exact::gemv, and gates the compiled step equal to
the plain one (torch.compile(gcmp._step), compiled_eq_plain: experiments/speed_fair_kaggle.py:793-797). Here
torch.library.opcheck checks every exact:: op's schema, fake implementation and dispatch, and a TLinG-style step
(exact::gemv + the group epilogue y = shr(t, 28 - s) + b, speed_fair_kaggle.py:724-725, 735-738) is compiled with the
aot_eager backend, captured in a HIP graph and replayed; every replay equals the eager step.
"""
import numpy as np
import pytest
import torch

from exact_amd import ops, synth
from exact_amd.tables import exp_t, silu_t

pytestmark = pytest.mark.gpu
DEV = "cuda"
E = torch.ops.exact
rng = np.random.default_rng(91)


def dev(a, dt):
    return torch.tensor(np.ascontiguousarray(a), dtype=dt, device=DEV)


def gemv_inputs(N, K):
    x16 = dev(rng.integers(-32767, 32768, K), torch.int16)
    wT = dev(rng.integers(-127, 128, (N, K)), torch.int8)
    Mg = dev(rng.integers(1, 1 << 15, (N, K // 128)), torch.int64)
    return x16, wT, Mg


def op_samples():
    thr = dev(synth.thresholds().astype(np.int64), torch.int64).to(torch.int32)
    N, K = 192, 256
    wp, mp = ops.PackedLinear.alloc(N, K, DEV)
    ops.synth_linear(wp, mp, N, K, synth.key(6, "w"), synth.key(6, "m"), synth.M_LO, synth.M_HI, thr)
    H, KV, hd, Smax = 4, 2, 64, 24
    expt = dev(exp_t(), torch.int32)
    return [
        (E.gemv, gemv_inputs(320, 512)),
        (E.gemm_g128, (dev(rng.integers(-32767, 32768, (5, K)), torch.int16), 15, wp, mp, N)),
        (E.gemm_g128, (dev(rng.integers(-127, 128, (40, K)), torch.int8), 7, wp, mp, N)),
        (E.rmsnorm_qrow, (dev(rng.integers(-(1 << 36), 1 << 36, (3, 896)), torch.int64),
                          dev(rng.integers(1 << 15, 1 << 17, 896), torch.int64), 15)),
        (E.swiglu_qrow, (dev(rng.integers(-(1 << 40), 1 << 40, (2, 2 * 320)), torch.int64),
                         dev(rng.integers(0, 8, 2), torch.int32), dev(silu_t(), torch.int32), 15)),
        (E.attention, (dev(rng.integers(-32767, 32768, (2, H, hd)), torch.int16), dev(rng.integers(0, 4, (2, H)), torch.int32),
                       dev(rng.integers(-32767, 32768, (2, KV, Smax, hd)), torch.int16),
                       dev(rng.integers(0, 4, (2, KV, Smax)), torch.int32),
                       dev(rng.integers(-(1 << 29), 1 << 29, (2, KV, Smax, hd)), torch.int64),
                       dev([1, 0], torch.int32), dev([20, 5], torch.int32), expt, 8192)),
        (E.router_topk, (dev(rng.integers(-(1 << 40), 1 << 40, (4, 60)), torch.int64), dev(rng.integers(0, 8, 4), torch.int32),
                         expt, 4)),
        (E.logits_argmax, (dev(rng.integers(-(1 << 40), 1 << 40, (2, 5000)), torch.int64), dev(rng.integers(0, 8, 2), torch.int32))),
    ]


def test_opcheck_every_exact_op():
    """schema, fake tensor, autograd registration and aot dispatch checks of every custom op of the boundary"""
    for op, args in op_samples():
        torch.library.opcheck(op, args)


def tlin_step(x16, wT, Mg, s, b):
    """TLinG for one row (R == 1) with its group epilogue: raw = exact::gemv(x16, wT, Mg); y = shr(raw, 28 - s) + b"""
    raw = torch.ops.exact.gemv(x16, wT, Mg)
    n = 28 - s
    return ((raw + (torch.ones_like(raw) << (n - 1))) >> n) + b


def test_compiled_step_equals_plain_and_replays_in_a_graph():
    N, K = 3584, 3584
    x16, wT, Mg = gemv_inputs(N, K)
    b = dev(rng.integers(-(1 << 20), 1 << 20, N), torch.int64)
    s = 9
    plain = tlin_step(x16, wT, Mg, s, b)
    cstep = torch.compile(tlin_step, backend="aot_eager", fullgraph=True)
    compiled = cstep(x16, wT, Mg, s, b)
    torch.cuda.synchronize()
    assert torch.equal(compiled, plain)
    # capture the compiled step in a HIP graph and replay it several times, with eager work and synchronisation
    # between the replays; every replay must equal the eager result
    static_x = x16.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        cstep(static_x, wT, Mg, s, b)
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = cstep(static_x, wT, Mg, s, b)
    for rep in range(4):
        xn = dev(rng.integers(-32767, 32768, K), torch.int16)
        static_x.copy_(xn)
        g.replay()
        torch.cuda.synchronize()
        want = tlin_step(xn, wT, Mg, s, b)
        _ = (want * 3).sum()                 # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
