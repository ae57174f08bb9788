"""The boundary's torch custom ops (exact::gemv, exact::gemm_g128, exact::rmsnorm_qrow, exact::swiglu_qrow,
exact::attention, exact::router_topk, exact::logits_argmax) are registered with fake implementations whose output
shapes and dtypes follow the contracts; checked on meta tensors (no GPU, no library call)."""
import torch

from exact_amd import ops  # noqa: F401  (registers the ops)

M = dict(device="meta")


def test_ops_registered():
    for name in ("gemv", "gemm_g128", "rmsnorm_qrow", "swiglu_qrow", "attention", "router_topk", "logits_argmax"):
        assert hasattr(torch.ops.exact, name), name


def test_fake_shapes():
    E = torch.ops.exact
    x16 = torch.empty((5, 256), dtype=torch.int16, **M)
    wp, mp = torch.empty(4 * 2 * 8192, dtype=torch.int8, **M), torch.empty(4 * 2 * 64, dtype=torch.int16, **M)
    t = E.gemm_g128(x16, 15, wp, mp, 200)
    assert t.shape == (5, 200) and t.dtype == torch.int64
    y = E.gemv(torch.empty(256, dtype=torch.int16, **M), torch.empty((300, 256), dtype=torch.int8, **M),
               torch.empty((300, 2), dtype=torch.int64, **M))
    assert y.shape == (300,) and y.dtype == torch.int64
    xq, s = E.rmsnorm_qrow(torch.empty((3, 896), dtype=torch.int64, **M), torch.empty(896, dtype=torch.int64, **M), 7)
    assert xq.shape == (3, 896) and xq.dtype == torch.int8 and s.shape == (3,) and s.dtype == torch.int32
    hq, sh = E.swiglu_qrow(torch.empty((2, 2 * 1408), dtype=torch.int64, **M), torch.empty(2, dtype=torch.int32, **M),
                           torch.empty(8194, dtype=torch.int32, **M), 15)
    assert hq.shape == (2, 1408) and hq.dtype == torch.int16 and sh.dtype == torch.int32
    out = E.attention(torch.empty((2, 28, 128), dtype=torch.int16, **M), torch.empty((2, 28), dtype=torch.int32, **M),
                      torch.empty((2, 4, 64, 128), dtype=torch.int16, **M), torch.empty((2, 4, 64), dtype=torch.int32, **M),
                      torch.empty((2, 4, 64, 128), dtype=torch.int64, **M), torch.empty(2, dtype=torch.int32, **M),
                      torch.empty(2, dtype=torch.int32, **M), torch.empty(10242, dtype=torch.int32, **M), 5793)
    assert out.shape == (2, 28 * 128) and out.dtype == torch.int64
    p, e = E.router_topk(torch.empty((4, 60), dtype=torch.int64, **M), torch.empty(4, dtype=torch.int32, **M),
                         torch.empty(10242, dtype=torch.int32, **M), 4)
    assert p.shape == (4, 4) and p.dtype == torch.int64 and e.dtype == torch.int32
    lg, ids = E.logits_argmax(torch.empty((2, 1000), dtype=torch.int64, **M), torch.empty(2, dtype=torch.int32, **M))
    assert lg.shape == (2, 1000) and ids.shape == (2,) and ids.dtype == torch.int32
