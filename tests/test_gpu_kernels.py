"""GPU parity of the HIP kernels against the oracle (bit-exact)."""
import numpy as np
import pytest
import torch

import exact_oracle as O
from exact_amd import ops, synth
from exact_amd.ops import I8, I16, I32, I64, PackedLinear

pytestmark = pytest.mark.gpu
DEV = "cuda"
rng = np.random.default_rng(2024)


def dev(a, dt):
    return ops.np_to_dev(a, dt, DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def thr():
    return torch.tensor(synth.thresholds().astype(np.int64)).to(torch.int32).to(DEV)


def synth_lin(thr, seed, name, N, K):
    kw, km = synth.key(seed, name + ".w"), synth.key(seed, name + ".m")
    wp, mp = PackedLinear.alloc(N, K, DEV)
    ops.synth_linear(wp, mp, N, K, kw, km, synth.M_LO, synth.M_HI, thr)
    return PackedLinear(wp, mp, N, K), kw, km


def oracle_t(xq, w, M):
    acc = O.group_acc(xq.astype(np.int64), w)
    return (acc * M[:, None, :]).sum(0)


def test_synth_matches_numpy_generator_and_pack(thr):
    N, K = 200, 384
    lin, kw, km = synth_lin(thr, 7, "t", N, K)
    w = synth.weights_np(kw, N, K)
    M = synth.scales_np(km, N, K)
    wp2, mp2 = ops.pack_linear(dev(w, I8), dev(M, I16))
    assert torch.equal(lin.wp, wp2) and torch.equal(lin.mp, mp2)


@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R", [1, 2, 5, 8])
@pytest.mark.parametrize("N,K", [(64, 128), (200, 384), (896, 896), (4864, 896), (896, 4864), (1000, 1408)])
def test_gemv_small_shapes(thr, abits, R, N, K):
    lin, kw, km = synth_lin(thr, 11, f"g{N}x{K}", N, K)
    lim = (1 << abits) - 1
    xq = rng.integers(-lim, lim + 1, (R, K))
    xq[0, :3] = [lim, -lim, 0]
    t = ops.gemv_g128(dev(xq, I16 if abits == 15 else I8), abits, lin)
    exp = oracle_t(xq, synth.weights_np(kw, N, K), synth.scales_np(km, N, K))
    assert np.array_equal(host(t), exp)


@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R", [16, 17, 37, 46, 49, 130])
def test_gemm_rows(thr, abits, R):
    """One row chunk of the GEMV kernel (15 / 16 rows) and the GEMM kernels beyond."""
    N, K = 640, 512
    lin, kw, km = synth_lin(thr, 12, "gemm", N, K)
    lim = (1 << abits) - 1
    xq = rng.integers(-lim, lim + 1, (R, K))
    t = ops.gemm_g128(dev(xq, I16 if abits == 15 else I8), abits, lin)
    assert np.array_equal(host(t), oracle_t(xq, synth.weights_np(kw, N, K), synth.scales_np(km, N, K)))


@pytest.mark.parametrize("name,N,K", [("gateup", 18944, 3584), ("down", 3584, 18944)])
def test_prefill_gemm_full_shapes(thr, name, N, K):
    """The 2048-token prefill GEMMs at full size, A8 (the benchmark) and A16 (the spec): 40 whole output rows and
    64 whole output columns against numpy (every row block, column block and K split is covered)."""
    M_ = 2048
    lin, kw, km = synth_lin(thr, 72, name, N, K)
    w = synth.weights_np(kw, N, K)
    Mg = synth.scales_np(km, N, K)
    rows = np.sort(np.concatenate([[0, M_ - 1], rng.choice(M_, 38, replace=False)]))
    cols = np.sort(np.concatenate([[0, N - 1], rng.choice(N, 62, replace=False)]))
    for abits in (7, 15):
        lim = (1 << abits) - 1
        xq = rng.integers(-lim, lim + 1, (M_, K))
        t = host(ops.gemm_g128(dev(xq, I16 if abits == 15 else I8), abits, lin))
        assert np.array_equal(t[rows], oracle_t(xq[rows], w, Mg)), (name, abits, "rows")
        assert np.array_equal(t[:, cols], oracle_t(xq, w[:, cols], Mg[:, cols])), (name, abits, "cols")


@pytest.mark.parametrize("M_,N,K", [(2048, 8192, 384), (2000, 8000, 1664), (1024, 36864, 768)])
def test_multi_round_gemm_whole_output(thr, M_, N, K):
    """A8 GEMMs of more 256 x 128 tiles than CUs (blocks in several rounds), every output against numpy: 512 tiles
    of 3 groups, 504 tiles of 13 groups with a ragged last row block and column tile, 1152 tiles of 6."""
    lin, kw, km = synth_lin(thr, 73, f"ps{N}", N, K)
    w = synth.weights_np(kw, N, K)
    Mg = synth.scales_np(km, N, K)
    xq = rng.integers(-127, 128, (M_, K))
    print(f"multi-round GEMM {M_} x {N} x {K}", flush=True)
    t = host(ops.gemm_g128(dev(xq, I8), 7, lin))
    for c0 in range(0, N, 2048):
        assert np.array_equal(t[:, c0:c0 + 2048], oracle_t(xq, w[:, c0:c0 + 2048], Mg[:, c0:c0 + 2048])), (M_, N, K, c0)


@pytest.mark.parametrize("name,N,K", [("q", 3584, 3584), ("kv", 512, 3584), ("gate", 18944, 3584), ("down", 3584, 18944)])
@pytest.mark.parametrize("R", [1, 2, 8])
def test_gemv_7b_shapes(thr, name, N, K, R):
    """Full Qwen2.5-7B GEMV shapes, x int8 U[-127, 127] (A8) and int16 (A16), bit-exact vs numpy."""
    lin, kw, km = synth_lin(thr, 70, name, N, K)
    w = synth.weights_np(kw, N, K)
    M = synth.scales_np(km, N, K)
    for abits in (7, 15):
        lim = (1 << abits) - 1
        xq = rng.integers(-lim, lim + 1, (R, K))
        t = ops.gemv_g128(dev(xq, I16 if abits == 15 else I8), abits, lin)
        assert np.array_equal(host(t), oracle_t(xq, w, M)), (name, R, abits)


def test_gemv_7b_head_rows(thr):
    """lm_head 152064 x 3584: all rows computed on the GPU, checked on the first and last 4096 rows."""
    N, K = 152064, 3584
    lin, kw, km = synth_lin(thr, 71, "head", N, K)
    M = synth.scales_np(km, N, K)
    for abits, R in ((7, 1), (15, 8)):
        lim = (1 << abits) - 1
        xq = rng.integers(-lim, lim + 1, (R, K))
        t = host(ops.gemv_g128(dev(xq, I16 if abits == 15 else I8), abits, lin))
        for n0, n1 in ((0, 4096), (N - 4096, N)):
            exp = oracle_t(xq, synth.weights_np(kw, N, K, n0, n1), M[:, n0:n1])
            assert np.array_equal(t[:, n0:n1], exp)


def test_requant_and_qrow_and_irms():
    R, N = 5, 3000
    t = rng.integers(-(1 << 50), 1 << 50, (R, N))
    s = rng.integers(0, 30, R).astype(np.int32)
    b = rng.integers(-1000, 1000, N)
    y = host(ops.requant_group(dev(t, I64), dev(s, I32), dev(b, I64)))
    assert np.array_equal(y, O.round_shift(t, 28 - s[:, None].astype(np.int64)) + b)
    x = rng.integers(-(1 << 40), 1 << 40, (R, 2048)) >> rng.integers(0, 40, (R, 1))
    for bits in (15, 7):
        xq, sq = ops.qrow(dev(x, I64), bits)
        exq, es = O.qrow(x, bits)
        assert np.array_equal(host(xq).astype(np.int64), exq) and np.array_equal(host(sq), es[:, 0])
    g = synth.vector_np(synth.key(1, "g"), 2048, *synth.GAIN)
    assert np.array_equal(host(ops.irms(dev(x, I64), dev(g, I64))), O.irms(x, g))


def test_requant_channel_drop_rule():
    R, N = 4, 700
    acc = rng.integers(-(1 << 45), 1 << 45, (R, N))
    acc[1] >>= 30
    M = rng.integers(1 << 20, 1 << 26, N)
    s = rng.integers(0, 20, R).astype(np.int32)
    b = rng.integers(-100, 100, N)
    Mbits = int(M.max()).bit_length()
    y = host(ops.requant_channel(dev(acc, I64), dev(s, I32), dev(M, I64), Mbits, dev(b, I64)))
    assert np.array_equal(y, O.requant_channel(acc, s[:, None].astype(np.int64), M, Mbits, b))


def test_lut_nonlinearities_and_softmax():
    from exact_amd.tables import exp_t, silu_t, sig_t
    x = np.concatenate([rng.integers(-(20 << 16), 20 << 16, 50000), [-(16 << 16) - 1, -(16 << 16), (16 << 16) - 1, 16 << 16]])
    silu, sig, ex = dev(silu_t(), I32), dev(sig_t(), I32), dev(exp_t(), I32)
    assert np.array_equal(host(ops.isilu(dev(x, I64), silu)), O.isilu(x))
    assert np.array_equal(host(ops.isig(dev(x, I64), sig)), O.isig(x))
    sc = rng.integers(-(1 << 24), 1 << 24, (6, 300))
    nv = np.array([300, 1, 17, 299, 150, 64], np.int32)
    p = host(ops.isoftmax(dev(sc, I64), ex, dev(nv, I32)))
    valid = np.arange(300)[None, :] < nv[:, None]
    assert np.array_equal(p, O.isoftmax(sc, valid))


def test_logits_argmax_first_max_across_slices():
    """Multi-slice argmax keeps numpy's first maximum: ties inside a slice, across slices, at slice edges."""
    R, N = 5, 152064
    t = rng.integers(-(1 << 40), 1 << 40, (R, N))
    s = rng.integers(8, 16, R).astype(np.int32)
    lg = O.round_shift(t, 28 - s[:, None].astype(np.int64))
    top = lg.max() + (1 << 30)
    for r, cols in enumerate([(4095, 4096), (100000, 7), (152063,), (0, 152063), (4096, 8191, 8192)]):
        for c in cols:
            t[r, c] = top << (28 - int(s[r]))
    lg = O.round_shift(t, 28 - s[:, None].astype(np.int64))
    td, ids = dev(t, I64), torch.zeros(R, dtype=I32, device=DEV)
    out = torch.zeros((R, N), dtype=I64, device=DEV)
    ops.logits_argmax(td, dev(s, I32), out, ids, clear=True)
    assert np.array_equal(host(out), lg)
    assert host(ids).tolist() == lg.argmax(-1).tolist()
    assert not host(td).any()


def test_quant_rows_from_partial_maxima():
    R, K, ld = 3, 5000, 5120
    x = rng.integers(-(1 << 40), 1 << 40, (R, ld))
    x[1] >>= 30                                    # a row with a small shift
    x[2] = 0                                       # an all-zero row: s = 0
    nparts = 7
    part = np.zeros((R, nparts), np.int64)
    for r in range(R):                             # any split of the row into parts gives the same maximum
        for i, chunk in enumerate(np.array_split(np.abs(x[r, :K]), nparts)):
            part[r, i] = O.bitlen(chunk.max())
    xd = dev(x, I64)
    xq, sq = torch.zeros((R, K), dtype=torch.int16, device=DEV), torch.zeros(R, dtype=I32, device=DEV)
    ops.quant_rows(xd, dev(part, I32), nparts, 15, xq, sq, K=K, clear=True)
    eq, es = O.qrow(x[:, :K], 15)
    assert np.array_equal(host(xq).astype(np.int64), eq) and np.array_equal(host(sq), es[:, 0])
    assert not host(xd)[:, :K].any() and np.array_equal(host(xd)[:, K:], x[:, K:])


@pytest.mark.parametrize("R,I,bits", [(3, 4864, 15), (2, 18944, 15), (5, 1408, 7), (2, 24576, 15), (4, 100, 15)])
def test_swiglu_qrow(R, I, bits):
    """One-workgroup rows (I <= 20480) and the two-kernel slice path (longer rows); both leave t zeroed."""
    from exact_amd.tables import silu_t
    t = rng.integers(-(1 << 44), 1 << 44, (R, 2 * I))
    s = rng.integers(10, 20, R).astype(np.int32)
    td = dev(t, I64)
    hq, sh = ops.swiglu_qrow(td, dev(s, I32), dev(silu_t(), I32), bits=bits, clear=True)
    g = O.round_shift(t[:, :I], 28 - s[:, None].astype(np.int64))
    u = O.round_shift(t[:, I:], 28 - s[:, None].astype(np.int64))
    eq, es = O.qrow(O.round_shift(O.isilu(g) * u, 16), bits)
    assert np.array_equal(host(hq).astype(np.int64), eq) and np.array_equal(host(sh), es[:, 0])
    assert not host(td).any()
    # with an h scratch and no clear, t stays as it was (trace capture) and the result is the same
    td = dev(t, I64)
    h = torch.full((R, I), -3, dtype=I64, device=DEV)
    hq, sh = ops.swiglu_qrow(td, dev(s, I32), dev(silu_t(), I32), bits=bits, clear=False, h=h)
    assert np.array_equal(host(hq).astype(np.int64), eq) and np.array_equal(host(sh), es[:, 0])
    assert np.array_equal(host(td), t)



@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R,N,K,mbits", [(1, 3584, 3584, 21), (5, 896, 4864, 27), (16, 500, 1408, 30), (46, 640, 896, 22),
                                         (130, 1000, 2048, 21)])
def test_wide_group_scales(abits, R, N, K, mbits):
    """Group scales beyond int16 (quantised checkpoints give M up to about 2^21; the reference allows < 2^27) as two
    planes M = mh * 2^15 + low: GEMV, chunked GEMV and GEMM (A8, and A16 as digit rows) equal the int64 numpy sum
    (which wraps as the kernels do)."""
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    M = rng.integers(0, 1 << mbits, (K // 128, N))
    M[0, :3] = [0, (1 << 15) - 1, 1 << 15]
    lin = ops.pack_group_linear(w, M, DEV)
    assert lin.mh is not None
    lim = (1 << abits) - 1
    xq = rng.integers(-lim, lim + 1, (R, K))
    xq[0, :2] = [lim, -lim]
    t = ops.linear_t(dev(xq, I16 if abits == 15 else I8), abits, lin)
    assert np.array_equal(host(t), oracle_t(xq, w, M)), (R, abits)


@pytest.mark.parametrize("R", [15, 16, 45])
def test_wide_scales_a16_generic_gemm_entry_row_chunks(R):
    """The generic GEMM entry (the one INTEGRATION.md binds for TLinG's R > 1 branch) with int16 rows and wide scales
    runs GEMV row chunks of 15 up to 3 x 15 rows and equals the int64 sum."""
    K, N = 1408, 500
    w = rng.integers(-127, 128, (K, N)).astype(np.int8)
    M = rng.integers(1 << 15, 1 << 21, (K // 128, N))
    lin = ops.pack_group_linear(w, M, DEV)
    assert lin.mh is not None
    xq = rng.integers(-32767, 32768, (R, K))
    t = torch.zeros((R, N), dtype=I64, device=DEV)
    ops._linear("exact_gemm_g128", dev(xq, I16), 15, lin, t)
    assert np.array_equal(host(t), oracle_t(xq, w, M))


def test_wide_scales_a16_generic_gemm_entry_is_refused():
    """The generic GEMM entry with int16 rows above 3 x 15 has no wide-scale kernel: it returns 'unsupported' (the
    digit-row entry, which ops uses, covers it)."""
    K, N, R = 256, 64, 46
    lin = ops.pack_group_linear(rng.integers(-127, 128, (K, N)).astype(np.int8), rng.integers(1 << 15, 1 << 20, (2, N)), DEV)
    x = dev(rng.integers(-100, 100, (R, K)), I16)
    with pytest.raises(ops.ExactError, match="unsupported"):
        ops._linear("exact_gemm_g128", x, 15, lin, None)


@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R,N,K,slice_", [(1, 3584, 3584, 128), (3, 896, 896, 64), (15, 512, 18944, 1024), (2, 5120, 13824, 1024),
                                         (1, 2048, 2048, 128)])
def test_gemv_qrow_acc(thr, abits, R, N, K, slice_):
    """qrow folded into the consuming GEMV: t += qrow(xs).W with the row shifts from slice bit lengths equals the
    oracle's qrow then linear totals; the shifts come back in s_out; t accumulates onto what it held."""
    if abits == 7 and R > 16 or abits == 15 and R > 15:
        pytest.skip("beyond the GEMV rows")
    lin, kw, km = synth_lin(thr, 91, "xq", N, K)
    w, M = synth.weights_np(kw, N, K), synth.scales_np(km, N, K)
    ldx = K + 256
    xs = rng.integers(-(1 << 40), 1 << 40, (R, ldx)) >> rng.integers(0, 38, (R, 1))
    xs[0, 5] = 0
    nparts = -(-K // slice_)
    part = np.array([[O.bitlen(np.array([np.abs(xs[r, i * slice_:min(K, (i + 1) * slice_)]).max()]))[0]
                      for i in range(nparts)] for r in range(R)], np.int32)
    xq, s = O.qrow(xs[:, :K], abits)
    base = rng.integers(-(1 << 50), 1 << 50, (R, N))
    t = dev(base, I64)
    s_out = torch.full((R,), -1, dtype=I32, device=DEV)
    ops.gemv_qrow_acc(dev(xs, I64), dev(part, I32), nparts, abits, lin, t, s_out)
    assert np.array_equal(host(s_out), s[:, 0])
    assert np.array_equal(host(t), base + oracle_t(xq, w, M))


def test_swiglu_part_then_qrow_gemv_matches_swiglu_qrow(thr):
    """SwiGLU slices without the qrow (h and slice bit lengths) feeding gemv_qrow_acc give the same totals and shift
    as swiglu_qrow + GEMV, and leave the gate|up totals zeroed with clear."""
    from exact_amd.tables import silu_t
    R, I, D = 2, 18944, 3584
    lin, kw, km = synth_lin(thr, 92, "down", D, I)
    w, M = synth.weights_np(kw, D, I), synth.scales_np(km, D, I)
    tg = rng.integers(-(1 << 44), 1 << 44, (R, 2 * I))
    s = rng.integers(10, 20, R).astype(np.int32)
    td = dev(tg, I64)
    h = torch.empty((R, I), dtype=I64, device=DEV)
    part = torch.empty(R * -(-I // 1024), dtype=I32, device=DEV)
    ops.swiglu_part(td, dev(s, I32), dev(silu_t(), I32), h, part, clear=True)
    t = torch.zeros((R, D), dtype=I64, device=DEV)
    sh = torch.empty(R, dtype=I32, device=DEV)
    ops.gemv_qrow_acc(h, part, -(-I // 1024), 15, lin, t, sh)
    g = O.round_shift(tg[:, :I], 28 - s[:, None].astype(np.int64))
    u = O.round_shift(tg[:, I:], 28 - s[:, None].astype(np.int64))
    eq, es = O.qrow(O.round_shift(O.isilu(g) * u, 16), 15)
    assert np.array_equal(host(sh), es[:, 0])
    assert np.array_equal(host(t), oracle_t(eq, w, M))
    assert not host(td).any()


@pytest.mark.parametrize("R,I,K", [(1, 18944, 1792), (2, 4864, 896), (4, 13824, 640), (3, 128, 256), (1, 64, 128),
                                   (8, 1280, 384), (5, 128, 256), (7, 192, 128)])
def test_gemv_swiglu_matches_oracle(thr, R, I, K):
    """The gate|up GEMV with the SwiGLU in its epilogue: h is the oracle's SwiGLU of the gate|up totals, part the bit
    length of max |h| per 32 columns, t (when given) the totals; h and part feeding gemv_qrow_acc give the oracle's
    qrow shift and down totals. Row shifts s put row 0's gate values inside the SiLU table's +-16 range (interpolated
    entries) and the last row's far outside it (saturation). Rows 4 to 7 (R > 4) sit in the second 16-lane group of
    the matrix-core layout, each with its own bit lengths."""
    from exact_amd.tables import silu_t
    lin, kw, km = synth_lin(thr, 93, f"gu{I}x{K}", 2 * I, K)
    xq = rng.integers(-32767, 32768, (R, K))
    xq[0, :2] = [32767, -32767]
    if R > 1:
        xq[1] >>= 9
    t = oracle_t(xq, synth.weights_np(kw, 2 * I, K), synth.scales_np(km, 2 * I, K))
    bl = O.bitlen(np.abs(t).max(1))
    s = 28 - np.maximum(bl - 21, 0)
    s[-1] = 28 if R > 1 else s[-1]
    g = O.round_shift(t[:, :I], 28 - s[:, None])
    u = O.round_shift(t[:, I:], 28 - s[:, None])
    h_exp = O.round_shift(O.isilu(g) * u, 16)
    assert (np.abs(g[0]) < (16 << 16)).sum() > I // 4   # the table's interpolated range is exercised
    h = torch.full((R, I), -5, dtype=I64, device=DEV)
    pc = ops.SWIGLU_PART_COLS
    part = torch.full((R * (I // pc),), -1, dtype=I32, device=DEV)
    td = torch.full((R, 2 * I), 7, dtype=I64, device=DEV) if R == 2 else None
    ops.gemv_swiglu(dev(xq, I16), lin, dev(s.astype(np.int32), I32), dev(silu_t(), I32), h, part, t=td)
    assert np.array_equal(host(h), h_exp)
    part_exp = O.bitlen(np.abs(h_exp).reshape(R, I // pc, pc).max(2)).reshape(-1)
    assert np.array_equal(host(part), part_exp)
    if td is not None:
        assert np.array_equal(host(td), t)
    if I % 128:
        return   # a down linear needs whole 128-wide groups
    D = 192
    down, kw2, km2 = synth_lin(thr, 94, f"dn{I}", D, I)
    td2 = torch.zeros((R, D), dtype=I64, device=DEV)
    sh = torch.full((R,), -1, dtype=I32, device=DEV)
    ops.gemv_qrow_acc(h, part, I // pc, 15, down, td2, sh)
    eq, es = O.qrow(h_exp, 15)
    assert np.array_equal(host(sh), es[:, 0])
    assert np.array_equal(host(td2), oracle_t(eq, synth.weights_np(kw2, D, I), synth.scales_np(km2, D, I)))


def test_gemv_swiglu_refuses_unsupported_shapes(thr):
    """More than 8 rows, or I not a multiple of 64: 'unsupported' (the model keeps the GEMV + SwiGLU launches then)."""
    from exact_amd.tables import silu_t
    lin, _, _ = synth_lin(thr, 95, "gu_bad", 2 * 96, 128)
    st = dev(silu_t(), I32)
    for R in (9, 1):   # 9 rows; one row of I = 96
        with pytest.raises(ops.ExactError, match="unsupported"):
            ops.gemv_swiglu(dev(np.zeros((R, 128)), I16), lin, dev(np.full(R, 20), I32), st,
                            torch.zeros((R, 96), dtype=I64, device=DEV), torch.zeros(R * 96, dtype=I32, device=DEV))


@pytest.mark.parametrize("R", [20, 33, 47, 60, 100, 300])
def test_zeroed_gemm_entries_match(thr, R):
    """exact_gemm_g128_zeroed / _a16_zeroed on a zeroed t give the oracle's totals on every path: int8 and int16
    GEMV row chunks (R <= 48), the int16 digit-row GEMM and the int8 GEMM, with K splits (o-shaped N = 2048 leaves
    few tiles) and without."""
    for name, N, K in (("zo", 2048, 2048), ("zg", 4096, 512)):
        lin, kw, km = synth_lin(thr, 72, name, N, K)
        w = synth.weights_np(kw, N, K)
        M = synth.scales_np(km, N, K)
        for abits in (15, 7):
            lim = (1 << abits) - 1
            xq = rng.integers(-lim, lim + 1, (R, K))
            want = oracle_t(xq, w, M)
            t = torch.zeros((R, N), dtype=I64, device=DEV)
            ops.linear_t(dev(xq, I16 if abits == 15 else I8), abits, lin, t, zeroed=True)
            assert np.array_equal(host(t), want), (name, R, abits)


def test_producer_digit_rows_feed_the_digit_gemm(thr):
    """rmsnorm_qrow, quant_rows and swiglu_qrow with x8 write the int16 rows' digit rows exactly as the GEMM's own
    split does, and exact_gemm_g128_digits on them equals exact_gemm_g128_a16 on the int16 rows."""
    R, D, N = 64, 1024, 768
    lin, kw, km = synth_lin(thr, 73, "dg", N, D)
    want_split = lambda q: np.stack([q >> 8, (q & 255) - 128], 1).reshape(2 * R, -1)
    x = dev(rng.integers(-(1 << 40), 1 << 40, (R, D)), I64)
    g = dev(rng.integers(1 << 15, 1 << 17, D), I64)
    x8 = torch.zeros((2 * R, D), dtype=I8, device=DEV)
    xq, s = ops.rmsnorm_qrow(x.clone(), g, 15, x8=x8)
    q = host(xq).astype(np.int64)
    assert np.array_equal(host(x8), want_split(q))
    for zeroed in (False, True):
        t_d = torch.zeros((R, N), dtype=I64, device=DEV)
        ops.gemm_g128(xq, 15, lin, t_d, zeroed=zeroed, x8=x8)
        t_a = ops.gemm_g128(xq, 15, lin)
        assert np.array_equal(host(t_d), host(t_a))
    src = dev(rng.integers(-(1 << 40), 1 << 40, (R, 2048)), I64)
    part = dev(np.full((R, 2), 41), I32)
    aq = torch.zeros((R, 2048), dtype=I16, device=DEV)
    a8 = torch.zeros((2 * R, 2048), dtype=I8, device=DEV)
    ops.quant_rows(src, part, 2, 15, aq, torch.zeros(R, dtype=I32, device=DEV), x8=a8)
    assert np.array_equal(host(a8), want_split(host(aq).astype(np.int64)))
    from exact_amd.tables import silu_t
    silu = dev(silu_t(), I32)
    for I in (1408, 9000):   # one workgroup per row; slices over many workgroups
        t = dev(rng.integers(-(1 << 44), 1 << 44, (R, 2 * I)), I64)
        h8 = torch.zeros((2 * R, I), dtype=I8, device=DEV)
        hq, _ = ops.swiglu_qrow(t, dev(rng.integers(0, 8, R), I32), silu, 15, x8=h8)
        assert np.array_equal(host(h8), want_split(host(hq).astype(np.int64)))


@pytest.mark.parametrize("D", [896, 2048, 3584, 5120])
def test_rmsnorm_qrow_row_sizes(D):
    """residual + irms + qrow at the model row sizes (512-, 1024- and 768-thread blocks) against the oracle."""
    R = 3
    x = rng.integers(-(1 << 36), 1 << 36, (R, D))
    t = rng.integers(-(1 << 44), 1 << 44, (R, D))
    s = rng.integers(0, 12, R)
    g = rng.integers(1 << 15, 1 << 17, D)
    xd, td = dev(x, I64), dev(t, I64)
    xq, sq = ops.rmsnorm_qrow(xd, dev(g, I64), 15, td, dev(s, I32), clear=True)
    x2 = x + O.round_shift(t, (28 - s)[:, None])
    want_q, want_s = O.qrow(O.irms(x2, g), 15)
    assert np.array_equal(host(xd), x2)
    assert np.array_equal(host(xq), want_q) and np.array_equal(host(sq).reshape(-1), np.asarray(want_s).reshape(-1))
    assert not host(td).any()


def _norm_case(kind, R, K, rng_):
    """Residual rows x, residual totals and shifts for the norm-fused GEMV, from ordinary to the edges of the
    row program's bounds: x << 16 wrapping int64, rows of zeros and of tiny values, left-shifting residuals."""
    x = rng_.integers(-(1 << 30), 1 << 30, (R, K))
    res = rng_.integers(-(1 << 44), 1 << 44, (R, K))
    rs = rng_.integers(0, 20, R)
    if kind == "huge":                  # |x| near 2^62: x << 16 wraps, k reaches 38
        x = rng_.integers(-(1 << 62), 1 << 62, (R, K))
        res = np.zeros((R, K), np.int64)
    elif kind == "zeros":
        x = np.zeros((R, K), np.int64)
        res = np.zeros((R, K), np.int64)
    elif kind == "tiny":                # one nonzero element: the largest quotient the row program can meet
        x = np.zeros((R, K), np.int64)
        x[:, 7] = rng_.integers(1, 100, R)
        res = np.zeros((R, K), np.int64)
    elif kind == "leftshift":           # res_s above 28: the residual is shifted left
        rs = rng_.integers(29, 40, R)
        res = rng_.integers(-(1 << 20), 1 << 20, (R, K))
    return x, res, rs


@pytest.mark.parametrize("kind", ["plain", "huge", "zeros", "tiny", "leftshift", "nores"])
@pytest.mark.parametrize("R,N,K", [(1, 4608, 3584), (2, 1152, 896), (1, 7168, 5120), (2, 640, 2048), (1, 300, 6144), (2, 4608, 3584),
                                   (1, 6144, 2048), (2, 7168, 5120)])
def test_gemv_norm_acc(thr, kind, R, N, K):
    """exact_gemv_g128_norm_acc: x = x_in + rs(res_t, 28 - res_s), t += qrow(irms(x, g), 15) . W, x_out = x, s_out, xq_out,
    against the oracle's irms / qrow / group linear; t starts from a running total."""
    rng_ = np.random.default_rng(R * 1000 + K + len(kind))
    lin, kw, km = synth_lin(thr, 21, f"norm{K}", N, K)
    w, M = synth.weights_np(kw, N, K), synth.scales_np(km, N, K)
    x, res, rs = _norm_case(kind, R, K, rng_)
    g = rng_.integers(1 << 14, 1 << 17, K)
    g[::5] = -g[::5]
    xn = x if kind == "nores" else x + O.round_shift(res, (28 - rs)[:, None])
    xq, s = O.qrow(O.irms(xn, g), 15)
    t0 = rng_.integers(-(1 << 50), 1 << 50, (R, N))
    want = t0 + oracle_t(xq, w, M)
    td = dev(t0, I64)
    x_out = torch.full((R, K), 7, dtype=I64, device=DEV)
    s_out = torch.full((R,), -1, dtype=I32, device=DEV)
    xq_out = torch.zeros((R, K), dtype=I16, device=DEV)
    xd = dev(x, I64)
    ops.gemv_norm_acc(xd, None if kind == "nores" else dev(res, I64), None if kind == "nores" else dev(rs, I32), dev(g, I64),
                      lin, td, s_out, x_out=x_out, xq_out=xq_out)
    assert np.array_equal(host(xq_out), xq), kind
    assert np.array_equal(host(s_out), s[:, 0]), kind
    assert np.array_equal(host(x_out), xn), kind
    assert np.array_equal(host(td), want), kind
    assert np.array_equal(host(xd), x)      # the input rows are left as they were


@pytest.mark.parametrize("kind", ["plain", "huge", "zeros", "tiny", "leftshift", "nores"])
@pytest.mark.parametrize("R,I,K", [(1, 4864, 896), (2, 4864, 896), (1, 2816, 2048), (2, 640, 1024), (1, 64, 128),
                                   (1, 18944, 3584), (2, 13824, 5120), (1, 192, 2176)])
def test_gemv_norm_swiglu(thr, kind, R, I, K):
    """exact_gemv_g128_norm_swiglu: x = x_in + rs(res_t, 28 - res_s), xq, s = qrow(irms(x, g), 15), h = SwiGLU of the
    gate|up totals xq . W with the row shifts s, part = bit length of max |h| per 32 columns, t = the totals, x_out = x,
    s_out = s, against the oracle; h and part feed the quantising down GEMV as the unfused path's do. Rows wider than
    2048 run 8-wave blocks: 4 pairs x 2 k parts (the 7B's I = 18944) or 2 x 4 (the 14B's 13824, and I = 192)."""
    from exact_amd.tables import silu_t
    rng_ = np.random.default_rng(R * 1000 + K + I + len(kind))
    lin, kw, km = synth_lin(thr, 22, f"nsw{I}x{K}", 2 * I, K)
    w, M = synth.weights_np(kw, 2 * I, K), synth.scales_np(km, 2 * I, K)
    x, res, rs = _norm_case(kind, R, K, rng_)
    g = rng_.integers(1 << 14, 1 << 17, K)
    g[::5] = -g[::5]
    xn = x if kind == "nores" else x + O.round_shift(res, (28 - rs)[:, None])
    xq, s = O.qrow(O.irms(xn, g), 15)
    t = oracle_t(xq, w, M)
    gg = O.round_shift(t[:, :I], 28 - s)
    uu = O.round_shift(t[:, I:], 28 - s)
    h_exp = O.round_shift(O.isilu(gg) * uu, 16)
    pc = ops.SWIGLU_PART_COLS
    part_exp = O.bitlen(np.abs(h_exp).reshape(R, I // pc, pc).max(2)).reshape(-1)
    h = torch.full((R, I), -5, dtype=I64, device=DEV)
    part = torch.full((R * (I // pc),), -1, dtype=I32, device=DEV)
    td = torch.full((R, 2 * I), 7, dtype=I64, device=DEV)
    x_out = torch.full((R, K), 7, dtype=I64, device=DEV)
    s_out = torch.full((R,), -1, dtype=I32, device=DEV)
    xd = dev(x, I64)
    nores = kind == "nores"
    ops.gemv_norm_swiglu(xd, None if nores else dev(res, I64), None if nores else dev(rs, I32), dev(g, I64), lin, s_out,
                         dev(silu_t(), I32), h, part, x_out=x_out, t=td)
    assert np.array_equal(host(s_out), s[:, 0]), kind
    assert np.array_equal(host(x_out), xn), kind
    assert np.array_equal(host(td), t), kind
    assert np.array_equal(host(h), h_exp), kind
    assert np.array_equal(host(part), part_exp), kind
    assert np.array_equal(host(xd), x)      # the input rows are left as they were
    if I % 128:
        return
    D = 192
    down, kw2, km2 = synth_lin(thr, 23, f"nswd{I}", D, I)
    td2 = torch.zeros((R, D), dtype=I64, device=DEV)
    sh = torch.full((R,), -1, dtype=I32, device=DEV)
    ops.gemv_qrow_acc(h, part, I // pc, 15, down, td2, sh)
    eq, es = O.qrow(h_exp, 15)
    assert np.array_equal(host(sh), es[:, 0])
    assert np.array_equal(host(td2), oracle_t(eq, synth.weights_np(kw2, D, I), synth.scales_np(km2, D, I)))


def test_gemv_norm_swiglu_refuses_unsupported_shapes(thr):
    """More than 2 rows, rows wider than 8192, or I not a multiple of 64: 'unsupported'; x_out aliasing x_in: bad
    argument."""
    from exact_amd.tables import silu_t
    st = dev(silu_t(), I32)
    for R, I, K in ((3, 64, 128), (1, 64, 8320), (1, 96, 128)):
        lin, _, _ = synth_lin(thr, 24, f"nswbad{R}{I}{K}", 2 * I, K)
        with pytest.raises(ops.ExactError, match="unsupported"):
            ops.gemv_norm_swiglu(torch.zeros((R, K), dtype=I64, device=DEV), None, None,
                                 torch.ones(K, dtype=I64, device=DEV), lin, torch.zeros(R, dtype=I32, device=DEV), st,
                                 torch.zeros((R, I), dtype=I64, device=DEV), torch.zeros(R * I, dtype=I32, device=DEV))
    lin, _, _ = synth_lin(thr, 24, "nswalias", 128, 128)
    xin = torch.zeros((1, 128), dtype=I64, device=DEV)
    with pytest.raises(ops.ExactError, match="bad argument"):
        ops.gemv_norm_swiglu(xin, None, None, torch.ones(128, dtype=I64, device=DEV), lin,
                             torch.zeros(1, dtype=I32, device=DEV), st, torch.zeros((1, 64), dtype=I64, device=DEV),
                             torch.zeros(64, dtype=I32, device=DEV), x_out=xin)


@pytest.mark.parametrize("kind", ["plain", "huge", "zeros", "tiny", "leftshift"])
@pytest.mark.parametrize("D,bits", [(896, 15), (3584, 15), (5120, 15), (2048, 7), (100, 15)])
def test_rmsnorm_qrow_edges(kind, D, bits):
    """The standalone residual + irms + qrow kernel (in place, residual cleared, digit rows) on the same edge rows as
    the norm-fused GEMV, int16 and int8 quantisation, against the oracle."""
    R = 2
    rng_ = np.random.default_rng(D + bits + 17 * len(kind))
    x, res, rs = _norm_case(kind, R, D, rng_)
    g = rng_.integers(1 << 14, 1 << 17, D)
    g[1::7] = -g[1::7]
    xd, td = dev(x, I64), dev(res, I64)
    x8 = torch.zeros((2 * R, D), dtype=I8, device=DEV) if bits == 15 else None
    xq, sq = ops.rmsnorm_qrow(xd, dev(g, I64), bits, td, dev(rs, I32), clear=True, x8=x8)
    x2 = x + O.round_shift(res, (28 - rs)[:, None])
    want_q, want_s = O.qrow(O.irms(x2, g), bits)
    assert np.array_equal(host(xd), x2), kind
    assert np.array_equal(host(xq), want_q) and np.array_equal(host(sq).reshape(-1), np.asarray(want_s).reshape(-1)), kind
    assert not host(td).any()
    if x8 is not None:
        d8 = host(x8).astype(np.int64)
        assert np.array_equal(d8[0::2] * 256 + d8[1::2] + 128, want_q), kind


@pytest.mark.parametrize("R,N,K", [(1, 10001, 3456), (3, 9600, 3584), (16, 4100, 8192)])
def test_gemv_large_a8_partial_row_block(thr, R, N, K):
    """Large int8-row weights (the 1024-thread-block launch) with N not a multiple of 64, so the last row block is
    partial: overwrite and accumulate modes, bit-exact vs numpy."""
    lin, kw, km = synth_lin(thr, 73, f"bal{N}", N, K)
    xq = rng.integers(-127, 128, (R, K))
    exp = oracle_t(xq, synth.weights_np(kw, N, K), synth.scales_np(km, N, K))
    t = ops.gemv_g128(dev(xq, I8), 7, lin)
    assert np.array_equal(host(t), exp)
    t0 = rng.integers(-(1 << 40), 1 << 40, (R, N))
    acc = dev(t0, I64)
    ops.gemv_g128_acc(dev(xq, I8), 7, lin, acc)
    assert np.array_equal(host(acc), exp + t0)
