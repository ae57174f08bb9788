"""GPU parity of the mixture-of-experts path (MoEInt.moe, moe_exact_kaggle.py:454-467) against the oracle:
router top-k with ties, dispatch bookkeeping, the expert GEMV, the combination, and whole models."""
import numpy as np
import pytest
import torch

import exact_oracle as O
import helpers
from exact_amd import ops, synth
from exact_amd.model import DeviceWeights, GraphDecoder, TModel
from exact_amd.tables import DeviceTables

pytestmark = pytest.mark.gpu
DEV = "cuda"
I32, I64 = torch.int32, torch.int64


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def dev(a, dt):
    return torch.tensor(np.asarray(a), dtype=dt, device=DEV)


@pytest.fixture(scope="module")
def tab():
    return DeviceTables(DEV, 16, 64, 1e4)


@pytest.mark.parametrize("R,NE,k", [(1, 60, 4), (8, 60, 4), (37, 6, 2), (5, 64, 8), (3, 100, 6)])
def test_router_topk_matches_oracle(tab, R, NE, k):
    """Routers of up to 64 experts run one wave per row, wider ones a block (100 experts)."""
    rng = np.random.default_rng(R * 100 + NE)
    t = rng.integers(-(1 << 40), 1 << 40, (R, NE))
    # ties: copies of one logit inside a row, so equal probabilities must resolve to the lower index
    t[:, NE // 2] = t[:, 1]
    t[:, NE - 1] = t[:, 0]
    if R > 2:
        t[2] = t[2, 0]                                   # an all-equal row
    s = rng.integers(0, 20, R)
    # the router row as the fused router|gate GEMV leaves it: NE logits, padding, the gate logit at a 64 boundary
    gcol = -(-NE // 64) * 64
    tg = rng.integers(-(1 << 44), 1 << 44, R)
    tfull = np.zeros((R, gcol + 1), np.int64)
    tfull[:, :NE], tfull[:, gcol] = t, tg
    td = dev(tfull, I64)
    p_sel, e_sel = torch.zeros((R, k), dtype=I64, device=DEV), torch.zeros((R, k), dtype=I32, device=DEV)
    gate = torch.zeros(R, dtype=I64, device=DEV)
    ops.router_topk(td, dev(s, I32), tab.exp, k, p_sel, e_sel, clear=True, NE=NE, gate_col=gcol, sig=tab.sig, gate=gate)
    lg = O.round_shift(t, (28 - s)[:, None])
    p = O.isoftmax(lg, np.ones_like(lg, bool))
    sel = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    assert np.array_equal(host(e_sel), sel)
    assert np.array_equal(host(p_sel), np.take_along_axis(p, sel, -1))
    assert np.array_equal(host(gate), O.isig(O.round_shift(tg, 28 - s)))
    assert not host(td).any()                            # cleared for the next accumulating GEMV


@pytest.mark.parametrize("R,NE,k,ch", [(1, 60, 4, 15), (8, 60, 4, 15), (256, 60, 4, 15), (40, 6, 2, 16), (2048, 4, 2, 15),
                                      (100, 130, 8, 16), (2048, 60, 4, 128), (333, 60, 4, 256), (16, 4, 2, 3), (32, 2, 2, 5)])
def test_dispatch_groups_pairs_by_expert(R, NE, k, ch):
    """Up to 64 pairs run one wave (experts with several chunks at 16 x 2 and 32 x 2 pairs), more a block of 16."""
    rng = np.random.default_rng(R + NE)
    e_sel = np.stack([rng.choice(NE, k, replace=False) for _ in range(R)])
    s = rng.integers(0, 30, R)
    P = R * k
    nmax = ops.max_chunks(P, NE, ch)
    out = {n: torch.full((P,), -1, dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
    out.update({n: torch.full((nmax,), -1, dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
    out["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
    ops.moe_dispatch(dev(e_sel, I32), dev(s, I32), NE, k, ch, out)
    o = {n: host(v) for n, v in out.items()}
    q = np.arange(P)
    # stable grouping: positions sorted by (expert, pair index)
    order = np.lexsort((q, e_sel.reshape(-1)))
    assert np.array_equal(o["pidx"][order], q)
    assert np.array_equal(o["pair_row"][o["pidx"]], q // k)
    assert np.array_equal(o["s_pair"][o["pidx"]], s[q // k])
    n = int(o["nchunks"][0])
    assert n <= nmax
    covered = np.zeros(P, int)
    for c in range(n):
        e, p0, cnt = o["chunk_e"][c], o["chunk_p0"][c], o["chunk_n"][c]
        assert 1 <= cnt <= ch
        pairs = order[p0:p0 + cnt]
        assert (e_sel.reshape(-1)[pairs] == e).all()
        covered[p0:p0 + cnt] += 1
    assert (covered == 1).all()


@pytest.mark.parametrize("R,NE,k,ch", [(1, 60, 4, 4), (2, 60, 4, 15), (16, 4, 2, 3), (8, 64, 8, 5), (3, 7, 2, 1)])
def test_moe_route_matches_topk_and_dispatch(tab, R, NE, k, ch):
    """exact_moe_route (top-k and dispatch of decode rows in one wave): the oracle's top-k (ties to the lower expert),
    the gate and the cleared totals, the dispatch's stable grouping and chunks, and every output equal to
    exact_router_topk + exact_moe_dispatch; more than 64 experts or pairs are refused."""
    rng = np.random.default_rng(R * 7 + NE)
    t = rng.integers(-(1 << 40), 1 << 40, (R, NE))
    t[:, NE // 2] = t[:, 1]                              # ties inside a row
    if R > 1:
        t[1] = t[1, 0]                                   # an all-equal row
    s = rng.integers(0, 20, R)
    gcol = -(-NE // 64) * 64
    tfull = np.zeros((R, gcol + 1), np.int64)
    tfull[:, :NE], tfull[:, gcol] = t, rng.integers(-(1 << 44), 1 << 44, R)
    P, nmax = R * k, ops.max_chunks(R * k, NE, ch)

    def run(fused):
        td = dev(tfull, I64)
        p_sel, e_sel = torch.zeros((R, k), dtype=I64, device=DEV), torch.zeros((R, k), dtype=I32, device=DEV)
        gate = torch.zeros(R, dtype=I64, device=DEV)
        out = {n: torch.full((P,), -1, dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
        out.update({n: torch.full((nmax,), -1, dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
        out["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
        if fused:
            ops.moe_route(td, dev(s, I32), tab.exp, k, p_sel, e_sel, ch, out, clear=True, NE=NE, gate_col=gcol,
                          sig=tab.sig, gate=gate)
        else:
            ops.router_topk(td, dev(s, I32), tab.exp, k, p_sel, e_sel, clear=True, NE=NE, gate_col=gcol, sig=tab.sig,
                            gate=gate)
            ops.moe_dispatch(e_sel, dev(s, I32), NE, k, ch, out)
        return {"td": host(td), "p_sel": host(p_sel), "e_sel": host(e_sel), "gate": host(gate),
                **{n: host(v) for n, v in out.items()}}

    got, sep = run(True), run(False)
    for n in got:
        assert np.array_equal(got[n], sep[n]), n
    p = O.isoftmax(O.round_shift(t, (28 - s)[:, None]), np.ones((R, NE), bool))
    sel = np.argsort(-p, axis=-1, kind="stable")[:, :k]
    assert np.array_equal(got["e_sel"], sel) and np.array_equal(got["p_sel"], np.take_along_axis(p, sel, -1))
    assert not got["td"].any()
    q = np.arange(P)
    order = np.lexsort((q, sel.reshape(-1)))
    assert np.array_equal(got["pidx"][order], q)
    n = int(got["nchunks"][0])
    covered = np.zeros(P, int)
    for c in range(n):
        e, p0, cnt = got["chunk_e"][c], got["chunk_p0"][c], got["chunk_n"][c]
        assert 1 <= cnt <= ch and (sel.reshape(-1)[order[p0:p0 + cnt]] == e).all()
        covered[p0:p0 + cnt] += 1
    assert (covered == 1).all()
    if NE == 64:
        bad = torch.zeros((1, 65), dtype=I64, device=DEV)
        with pytest.raises(ops.ExactError, match="unsupported"):
            ops.moe_route(bad, dev(s[:1], I32), tab.exp, k, torch.zeros(k, dtype=I64, device=DEV),
                          torch.zeros(k, dtype=I32, device=DEV), ch,
                          {nm: torch.zeros(64, dtype=I32, device=DEV) for nm in
                           ("pidx", "pair_row", "s_pair", "chunk_e", "chunk_p0", "chunk_n", "nchunks")}, NE=65)


@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R,NE,k,N,K", [(1, 60, 4, 2816, 2048), (8, 60, 4, 2048, 1408), (50, 6, 2, 384, 256)])
def test_expert_gemv_matches_oracle(abits, R, NE, k, N, K):
    rng = np.random.default_rng(abits + R)
    lin = ops.ExpertLinears(NE, N, K, DEV)
    thr = dev(synth.thresholds().astype(np.int64), I64).to(I32)
    used = sorted(set(rng.choice(NE, min(NE, 2 * k + 2), replace=False).tolist()))
    e_sel = np.stack([rng.choice(used, k, replace=False) for _ in range(R)])
    ws, Ms = {}, {}
    for e in used:
        wp, mp = lin.part(e)
        kw, km = synth.key(7, f"e{e}.w"), synth.key(7, f"e{e}.m")
        ops.synth_linear(wp, mp, N, K, kw, km, synth.M_LO, synth.M_HI, thr)
        ws[e], Ms[e] = synth.weights_np(kw, N, K), synth.scales_np(km, N, K)
    lim = (1 << abits) - 1
    x = rng.integers(-lim, lim + 1, (R, K))
    P = R * k
    disp = {n: torch.zeros((P,), dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
    nmax = ops.max_chunks(P, NE, ops.chunk_rows(abits))
    disp.update({n: torch.zeros((nmax,), dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
    disp["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
    ops.moe_dispatch(dev(e_sel, I32), torch.zeros(R, dtype=I32, device=DEV), NE, k, ops.chunk_rows(abits), disp)
    xd = dev(x, torch.int16 if abits == 15 else torch.int8)
    t = torch.zeros((P, N), dtype=I64, device=DEV)
    ops.gemv_experts(xd, abits, disp["pair_row"], lin, disp, t)
    got = host(t)
    pidx = host(disp["pidx"])
    for q in range(P):
        r, e = q // k, e_sel.reshape(-1)[q]
        want = (O.group_acc(x[r:r + 1], ws[e]) * Ms[e][:, None, :]).sum(0)[0]
        assert np.array_equal(got[pidx[q]], want), (q, e)


def _expert_case(rng, abits, R, NE, k, N, K, used):
    lin = ops.ExpertLinears(NE, N, K, DEV)
    thr = dev(synth.thresholds().astype(np.int64), I64).to(I32)
    e_sel = np.stack([rng.choice(used, k, replace=False) for _ in range(R)])
    ws, Ms = {}, {}
    for e in range(NE):
        wp, mp = lin.part(e)
        kw, km = synth.key(9, f"e{e}.w"), synth.key(9, f"e{e}.m")
        ops.synth_linear(wp, mp, N, K, kw, km, synth.M_LO, synth.M_HI, thr)
        if e in used:
            ws[e], Ms[e] = synth.weights_np(kw, N, K), synth.scales_np(km, N, K)
    lim = (1 << abits) - 1
    return lin, e_sel, ws, Ms, rng.integers(-lim, lim + 1, (R, K))


def _dispatch(e_sel, NE, k, chunk, abits):
    R = e_sel.shape[0]
    P = R * k
    disp = {n: torch.zeros((P,), dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
    nmax = ops.max_chunks(P, NE, chunk)
    disp.update({n: torch.zeros((nmax,), dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
    disp["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
    ops.moe_dispatch(dev(e_sel, I32), torch.zeros(R, dtype=I32, device=DEV), NE, k, chunk, disp)
    return disp


@pytest.mark.parametrize("abits", [15, 7])
@pytest.mark.parametrize("R,NE,k,N,K,nused,full", [(64, 60, 4, 2816, 2048, 10, False), (17, 60, 4, 2048, 1408, 60, False),
                                                    (300, 3, 2, 384, 256, 3, True), (40, 6, 2, 200, 384, 6, True)])
def test_expert_gemm_matches_expert_gemv_and_oracle(abits, R, NE, k, N, K, nused, full):
    """The grouped matrix-core expert GEMM against the expert GEMV (oracle-pinned above) on every pair, and
    against the oracle on every pair (small shapes) or on 24 of them; (300, 3, 2) puts 200 pairs on each
    expert, so one expert spans several 128- and 256-pair chunks, and N = 200 leaves a ragged column tile."""
    rng = np.random.default_rng(100 * abits + R)
    used = sorted(rng.choice(NE, nused, replace=False).tolist())
    lin, e_sel, ws, Ms, x = _expert_case(rng, abits, R, NE, k, N, K, used)
    P = R * k
    xd = dev(x, torch.int16 if abits == 15 else torch.int8)
    dv = _dispatch(e_sel, NE, k, ops.chunk_rows(abits), abits)
    t_v = torch.zeros((P, N), dtype=I64, device=DEV)
    ops.gemv_experts(xd, abits, dv["pair_row"], lin, dv, t_v)
    dm = _dispatch(e_sel, NE, k, ops.EXPERT_CHUNK[abits], abits)
    assert np.array_equal(host(dm["pidx"]), host(dv["pidx"]))
    t_m = torch.full((P, N), -1, dtype=I64, device=DEV)   # every row is written, none accumulated
    ops.gemm_experts(xd, abits, dm["pair_row"], lin, dm, t_m, P)
    got = host(t_m)
    assert np.array_equal(got, host(t_v))
    pidx = host(dm["pidx"])
    qs = range(P) if full else rng.choice(P, 24, replace=False)
    for q in qs:
        r, e = q // k, e_sel.reshape(-1)[q]
        want = (O.group_acc(x[r:r + 1], ws[e]) * Ms[e][:, None, :]).sum(0)[0]
        assert np.array_equal(got[pidx[q]], want), (q, e)
    # pairs in dispatched order (row_map None): the expert down projection's input layout
    xs = xd[dm["pair_row"].long()].contiguous()
    t_d = torch.zeros((P, N), dtype=I64, device=DEV)
    ops.gemm_experts(xs, abits, None, lin, dm, t_d, P)
    assert np.array_equal(host(t_d), got)


def test_combine_matches_oracle(tab):
    rng = np.random.default_rng(5)
    R, k, D, NE = 6, 4, 512, 60
    x = rng.integers(-(1 << 30), 1 << 30, (R, D))
    P = R * k
    pidx = rng.permutation(P)
    t_ed = rng.integers(-(1 << 44), 1 << 44, (P, D))
    sh_pair = rng.integers(0, 26, P)
    p_sel = rng.integers(0, 1 << 20, (R, k))
    t_sd = rng.integers(-(1 << 44), 1 << 44, (R, D))
    sh_s = rng.integers(0, 26, R)
    gate = O.isig(rng.integers(-(20 << 16), 20 << 16, R))          # isig outputs in [0, 2^16]
    xd = dev(x, I64)
    args = [dev(a, dt) for a, dt in ((t_ed, I64), (sh_pair, I32), (p_sel, I64), (pidx, I32), (t_sd, I64), (sh_s, I32),
                                     (gate, I64))]
    ops.moe_combine(xd, args[0], args[1], args[2], args[3], k, args[4], args[5], args[6], clear=True)
    want = x.copy()
    for r in range(R):
        for j in range(k):
            q = pidx[r * k + j]
            ye = O.round_shift(t_ed[q], 28 - sh_pair[q])[None]
            want[r] += O.moe_weighted(p_sel, None, [r], j, ye)[0]     # the oracle's pinned expert weighting
        want[r] += O.round_shift(gate[r] * O.round_shift(t_sd[r], 28 - sh_s[r]), 16)
    assert np.array_equal(host(xd), want)
    assert not host(args[0]).any() and not host(args[4]).any()


@pytest.mark.parametrize("abits", [15, 7])
def test_tiny_moe_prefill_and_decode_match_oracle(abits):
    cfg = synth.CONFIGS["tiny-moe"]
    seed = 11
    om = helpers.oracle_model(cfg, seed, T=64, abits=abits)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64, abits=abits)
    ids = helpers.prompt(21, 24, cfg.V)
    stats = {}
    assert np.array_equal(host(tm.forward(ids)), om.forward(ids, stats=stats))
    assert len({int(e) for st in stats.values() for sel in st for e in sel.reshape(-1)}) > cfg.topk
    otoks, orows = O.greedy_decode(om, ids[:10], 5)
    cache = tm.new_cache(B=1)
    lg = host(tm.forward(ids[:10], cache))
    assert np.array_equal(lg[-1], orows[0])
    tok = int(lg[-1].argmax())
    for i in range(1, 5):
        lgi, nid = tm.decode_rows([tok], cache)
        assert np.array_equal(host(lgi)[0], orows[i]), i
        tok = int(host(nid)[0])
        assert tok == otoks[i]


@pytest.mark.parametrize("abits", [15, 7])
def test_tiny_moe_long_prefill_runs_grouped_expert_gemm(abits, monkeypatch):
    """A 60-token prefill (120 pairs) takes the grouped expert GEMM; logits equal the oracle's."""
    cfg = synth.CONFIGS["tiny-moe"]
    seed = 13
    om = helpers.oracle_model(cfg, seed, T=64, abits=abits)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64, abits=abits)
    calls = []
    real = ops.gemm_experts
    monkeypatch.setattr(ops, "gemm_experts", lambda *a: calls.append(a[-1]) or real(*a))
    ids = helpers.prompt(23, 60, cfg.V)
    assert np.array_equal(host(tm.forward(ids)), om.forward(ids))
    assert calls == [60 * cfg.topk] * (2 * cfg.NL)


def test_tiny_moe_batch_graph_decode_matches_oracle():
    cfg = synth.CONFIGS["tiny-moe"]
    seed = 12
    B = 3
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=48, batch=B)
    om = helpers.oracle_model(cfg, seed, T=48)
    prompts = [helpers.prompt(300 + b, 5 + 2 * b, cfg.V) for b in range(B)]
    cache = tm.new_cache()
    first = []
    for b, p in enumerate(prompts):
        first.append(int(host(tm.forward(p, cache, slot=b))[-1].argmax()))
    gd = GraphDecoder(tm, cache, B)
    gd.load(first)
    gd.capture()
    want = [O.greedy_decode(om, p, 4) for p in prompts]
    toks = [list(first)]
    for i in range(1, 4):
        lg, nid = gd.step()
        lgh = host(lg)
        for b in range(B):
            assert np.array_equal(lgh[b], want[b][1][i]), (i, b)
        toks.append(host(nid).tolist())
    for b in range(B):
        assert [t[b] for t in toks] == want[b][0][:4]


@pytest.mark.parametrize("R,NE,k,MI,K,D", [(1, 8, 4, 128, 256, 192), (2, 12, 4, 1408, 2048, 256), (8, 6, 4, 256, 384, 128),
                                           (3, 5, 2, 128, 128, 64)])
def test_fused_expert_gemvs_match_oracle(tab, R, NE, k, MI, K, D):
    """exact_gemv_g128_experts_swiglu + exact_gemv_g128_experts_qrow_acc (dispatched chunks of at most 4 pairs, so
    experts chosen by many rows split into several chunks): h of every (row, expert) pair is the oracle's SwiGLU of the
    pair's gate|up totals with the row's shift, part its bit lengths per 32 columns, and the down GEMV quantising h gives
    the oracle's qrow shift and expert down totals (moe_exact_kaggle.py:461-463)."""
    rng = np.random.default_rng(R * 100 + MI)
    thr = dev(synth.thresholds().astype(np.int64), I64).to(I32)
    gu, dn = ops.ExpertLinears(NE, 2 * MI, K, DEV), ops.ExpertLinears(NE, D, MI, DEV)
    used = sorted(rng.choice(NE, min(NE, k + 1), replace=False).tolist())
    e_sel = np.stack([rng.choice(used, k, replace=False) for _ in range(R)])
    wg, Mg, wd, Md = {}, {}, {}, {}
    for e in used:
        for lin, w, M, N, KK, tag in ((gu, wg, Mg, 2 * MI, K, "g"), (dn, wd, Md, D, MI, "d")):
            wp, mp = lin.part(e)
            kw, km = synth.key(31, f"{tag}{e}.w"), synth.key(31, f"{tag}{e}.m")
            ops.synth_linear(wp, mp, N, KK, kw, km, synth.M_LO, synth.M_HI, thr)
            w[e], M[e] = synth.weights_np(kw, N, KK), synth.scales_np(km, N, KK)
    x = rng.integers(-32767, 32768, (R, K))
    x[0, :2] = [32767, -32767]
    tot = {(r, e): (O.group_acc(x[r:r + 1], wg[e]) * Mg[e][:, None, :]).sum(0)[0] for r in range(R) for e in e_sel[r]}
    s = np.array([28 - max(int(O.bitlen(max(np.abs(tot[(r, e)]).max() for e in e_sel[r]))) - 21, 0) for r in range(R)])
    P = R * k
    disp = {n: torch.zeros((P,), dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
    nmax = ops.max_chunks(P, NE, ops.EXPERT_FUSE_CHUNK)
    disp.update({n: torch.zeros((nmax,), dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
    disp["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
    ops.moe_dispatch(dev(e_sel, I32), dev(s, I32), NE, k, ops.EXPERT_FUSE_CHUNK, disp)
    assert host(disp["chunk_n"])[:int(host(disp["nchunks"])[0])].max() <= ops.EXPERT_FUSE_CHUNK
    pc = ops.SWIGLU_PART_COLS
    h = torch.full((P, MI), -3, dtype=I64, device=DEV)
    part = torch.full((P * (MI // pc),), -1, dtype=I32, device=DEV)
    ops.gemv_experts_swiglu(dev(x, torch.int16), disp["pair_row"], gu, disp, disp["s_pair"], tab.silu, h, part)
    t = torch.zeros((P, D), dtype=I64, device=DEV)
    sh = torch.full((P,), -1, dtype=I32, device=DEV)
    ops.gemv_experts_qrow_acc(h, part, MI // pc, dn, disp, t, sh)
    gh, gp, gt, gs = host(h), host(part).reshape(P, MI // pc), host(t), host(sh)
    pidx = host(disp["pidx"])
    for q in range(P):
        r, e = q // k, e_sel.reshape(-1)[q]
        tt = tot[(r, e)]
        g = O.round_shift(tt[:MI], 28 - int(s[r]))
        u = O.round_shift(tt[MI:], 28 - int(s[r]))
        hv = O.round_shift(O.isilu(g) * u, 16)
        p = pidx[q]
        assert np.array_equal(gh[p], hv), (q, e)
        assert np.array_equal(gp[p], O.bitlen(np.abs(hv).reshape(MI // pc, pc).max(1))), (q, e)
        hq, hs = O.qrow(hv[None, :], 15)
        assert gs[p] == hs[0, 0], (q, e)
        assert np.array_equal(gt[p], (O.group_acc(hq, wd[e]) * Md[e][:, None, :]).sum(0)[0]), (q, e)


@pytest.mark.parametrize("R,NE,k,MI,SI,K,D", [(1, 60, 4, 1408, 5632, 2048, 2048), (2, 8, 4, 128, 512, 256, 192),
                                              (1, 6, 2, 256, 384, 384, 128)])
def test_moe_pairs_match_the_separate_launches(tab, R, NE, k, MI, SI, K, D):
    """exact_moe_swiglu_pair = exact_gemv_g128_experts_swiglu + exact_gemv_g128_swiglu (the shared expert on the same
    rows) and exact_moe_qrow_pair = exact_gemv_g128_experts_qrow_acc + exact_gemv_g128_qrow_acc (with its clearing
    range): every output equal to the separate launches' (those are pinned against the oracle above and in the
    whole-model tests), at the Qwen1.5-MoE-A2.7B shapes and smaller ones."""
    from exact_amd.ops import PackedLinear
    rng = np.random.default_rng(R * 1000 + MI + SI)
    thr = dev(synth.thresholds().astype(np.int64), I64).to(I32)
    gu, dn = ops.ExpertLinears(NE, 2 * MI, K, DEV), ops.ExpertLinears(NE, D, MI, DEV)
    used = sorted(rng.choice(NE, min(NE, k + 1), replace=False).tolist())
    for e in used:
        for lin, N, KK, tag in ((gu, 2 * MI, K, "g"), (dn, D, MI, "d")):
            wp, mp = lin.part(e)
            ops.synth_linear(wp, mp, N, KK, synth.key(41, f"{tag}{e}.w"), synth.key(41, f"{tag}{e}.m"), synth.M_LO, synth.M_HI,
                             thr)

    def packed(N, KK, tag):
        wp, mp = PackedLinear.alloc(N, KK, DEV)
        ops.synth_linear(wp, mp, N, KK, synth.key(43, tag + ".w"), synth.key(43, tag + ".m"), synth.M_LO, synth.M_HI, thr)
        return PackedLinear(wp, mp, N, KK)
    sgu, sdn = packed(2 * SI, K, "sgu"), packed(D, SI, "sd")
    e_sel = np.stack([rng.choice(used, k, replace=False) for _ in range(R)])
    x = dev(rng.integers(-32767, 32768, (R, K)), torch.int16)
    s = dev(rng.integers(0, 8, R), I32)
    P = R * k
    disp = {n: torch.zeros((P,), dtype=I32, device=DEV) for n in ("pidx", "pair_row", "s_pair")}
    nmax = ops.max_chunks(P, NE, ops.EXPERT_FUSE_CHUNK)
    disp.update({n: torch.zeros((nmax,), dtype=I32, device=DEV) for n in ("chunk_e", "chunk_p0", "chunk_n")})
    disp["nchunks"] = torch.zeros(1, dtype=I32, device=DEV)
    ops.moe_dispatch(dev(e_sel, I32), s, NE, k, ops.EXPERT_FUSE_CHUNK, disp)
    pc = ops.SWIGLU_PART_COLS
    outs = []
    for paired in (False, True):
        eh = torch.full((P, MI), -3, dtype=I64, device=DEV)
        ep = torch.full((P * (MI // pc),), -1, dtype=I32, device=DEV)
        sh = torch.full((R, SI), -5, dtype=I64, device=DEV)
        sp = torch.full((R * (SI // pc),), -1, dtype=I32, device=DEV)
        et, st = torch.zeros((P, D), dtype=I64, device=DEV), torch.zeros((R, D), dtype=I64, device=DEV)
        es, ss = torch.full((P,), -1, dtype=I32, device=DEV), torch.full((R,), -1, dtype=I32, device=DEV)
        zero = torch.full((333,), 9, dtype=I64, device=DEV)
        if paired:
            ops.moe_swiglu_pair(x, disp["pair_row"], gu, disp, disp["s_pair"], tab.silu, eh, ep, sgu, s, sh, sp)
            ops.moe_qrow_pair(eh, ep, MI // pc, dn, disp, et, es, sh, sp, SI // pc, sdn, st, ss, zero=zero)
        else:
            ops.gemv_experts_swiglu(x, disp["pair_row"], gu, disp, disp["s_pair"], tab.silu, eh, ep)
            ops.gemv_swiglu(x, sgu, s, tab.silu, sh, sp)
            ops.gemv_experts_qrow_acc(eh, ep, MI // pc, dn, disp, et, es)
            ops.gemv_qrow_acc(sh, sp, SI // pc, 15, sdn, st, ss, zero=zero)
        outs.append([host(v) for v in (eh, ep, sh, sp, et, es, st, ss, zero)])
    for a, b, name in zip(outs[0], outs[1], ("eh", "epart", "sh", "spart", "et", "es", "st", "ss", "zero")):
        assert np.array_equal(a, b), name
    assert not outs[1][8].any()
