"""GPU model parity: logits and greedy tokens bit-identical to the oracle (and to the reference's golden)."""
import os

import numpy as np
import pytest
import torch

import exact_oracle as O
import helpers
from exact_amd import ops, synth
from exact_amd._lib import ExactError
from exact_amd.model import DeviceWeights, GraphDecoder, TModel

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "intmodel_tiny.npz")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_golden_reference_intmodel_per_channel():
    """The reference's own IntModel logits and receipts (tests/golden/make_golden.py), per-channel mode."""
    z = np.load(GOLD)
    cfg_d = eval(bytes(z["cfg_json"]).decode(), {})
    cfg = synth.ModelConfig("golden", D=cfg_d["D"], H=cfg_d["H"], KV=cfg_d["KV"], hd=cfg_d["hd"], I=cfg_d["I"],
                            V=cfg_d["V"], NL=cfg_d["NL"], theta=cfg_d["theta"])
    arrays = {k: z[k] for k in z.files}
    arrays["emb"] = z["emb"].astype(np.int64)
    w = DeviceWeights.from_arrays(cfg, arrays, DEV, mode="channel")
    tm = TModel(w, Smax=cfg_d["T"])
    lg = host(tm.forward(z["prompt"].tolist()))
    assert np.array_equal(lg, z["logits"])
    # greedy continuation with the KV cache equals the oracle's (which equals the reference's generate)
    om = O.Model({"emb": arrays["emb"], "gf": z["gf"], "head": O.Lin(z["head.w"], z["head.M"], mode="channel"),
                  "layers": [dict(g1=z[f"{i}.g1"], g2=z[f"{i}.g2"],
                                  **{k: O.Lin(z[f"{i}.{k}.w"], z[f"{i}.{k}.M"], z[f"{i}.{k}.b"] if f"{i}.{k}.b" in z else None,
                                              mode="channel") for k in ("q", "k", "v", "o", "gate", "up", "down")})
                             for i in range(cfg.NL)]}, cfg_d)
    toks, rows = O.greedy_decode(om, z["prompt"].tolist(), 5)
    cache = tm.new_cache(B=1)
    lg = tm.forward(z["prompt"].tolist(), cache)
    tok = int(host(lg)[-1].argmax())
    got = [tok]
    for _ in range(4):
        lg, ids = tm.decode_rows([tok], cache)
        tok = int(host(ids)[0])
        got.append(tok)
    assert got == toks


@pytest.mark.parametrize("name", ["tiny", "tiny-tied"])
def test_synthetic_prefill_and_decode_match_oracle(name):
    cfg = synth.CONFIGS[name]
    seed = 3
    om = helpers.oracle_model(cfg, seed, T=128)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=128)
    ids = helpers.prompt(9, 20, cfg.V)
    assert np.array_equal(host(tm.forward(ids)), om(ids))
    # prefill 12 tokens then 6 greedy decode steps through the cache
    otoks, orows = O.greedy_decode(om, ids[:12], 6)
    cache = tm.new_cache(B=1)
    lg = host(tm.forward(ids[:12], cache))
    assert np.array_equal(lg[-1], orows[0])
    tok = int(lg[-1].argmax())
    for i in range(1, 6):
        lgi, nid = tm.decode_rows([tok], cache)
        assert np.array_equal(host(lgi)[0], orows[i]), i
        tok = int(host(nid)[0])
        assert tok == otoks[i]


@pytest.mark.parametrize("qkv_norm", [True, False])
@pytest.mark.parametrize("name", ["tiny", "tiny-hd128"])
def test_decode_with_swiglu_in_the_gate_up_gemv_matches_oracle(name, qkv_norm):
    """Decode rows of hidden sizes above 2048 (the fully norm-fused GEMVs off): the attention norm inside the q|k|v GEMV
    (qkv_norm, the residual alternating between two buffers) or a launch of its own, the FFN norm a launch of its own;
    the gate|up GEMV applies the SwiGLU in its epilogue and the down GEMV quantises its per-64-column bit lengths.
    Logits and greedy tokens equal the oracle's, eagerly and through the graph; a 2-token prefill takes the same
    path."""
    cfg = synth.CONFIGS[name]
    seed = 5
    om = helpers.oracle_model(cfg, seed, T=64)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64)
    tm.NORM_FUSE_D = 0
    tm.QKV_NORM = qkv_norm
    ids = helpers.prompt(11, 14, cfg.V)
    otoks, orows = O.greedy_decode(om, ids[:10], 6)
    cache = tm.new_cache(B=1)
    lg = host(tm.forward(ids[:8], cache))
    lg = host(tm.forward(ids[8:10], cache))        # 2 prefill rows: q|k|v epilogue apart, SwiGLU in the GEMV
    assert np.array_equal(lg[-1], orows[0])
    tok = int(lg[-1].argmax())
    for i in range(1, 4):
        lgi, nid = tm.decode_rows([tok], cache)
        assert np.array_equal(host(lgi)[0], orows[i]), i
        tok = int(host(nid)[0])
        assert tok == otoks[i]
    gd = GraphDecoder(tm, cache, 1)
    gd.load([tok])
    gd.capture()
    for i in range(4, 6):
        lgi, nid = gd.step()
        assert np.array_equal(host(lgi)[0], orows[i]), i
        tok = int(host(nid)[0])
        assert tok == otoks[i]


@pytest.mark.parametrize("name", ["tiny-hd128", "tiny"])
def test_chunked_prefill_on_matrix_core_attention_matches_oracle(name, monkeypatch):
    """hd 128 and hd 64: prompt chunks of TModel.PREFILL_MIN_ROWS[hd] rows or more take the matrix-core attention
    (exact_attention_prefill), here a prompt of 2 c tokens (c = that threshold + 4) as one chunk and as chunks of
    c + c, the second continuing the cache (start position c), then greedy decode steps."""
    cfg = synth.CONFIGS[name]
    c = TModel.PREFILL_MIN_ROWS[cfg.hd] + 4
    calls = []
    real = ops.attention_prefill
    monkeypatch.setattr(ops, "attention_prefill", lambda *a, **k: calls.append(a[5]) or real(*a, **k))
    seed = 4
    om = helpers.oracle_model(cfg, seed, T=2 * c + 24)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=2 * c + 24)
    ids = helpers.prompt(17, 2 * c, cfg.V)
    want = om(ids)
    assert np.array_equal(host(tm.forward(ids)), want)
    cache = tm.new_cache(B=1)
    lg1 = host(tm.forward(ids[:c], cache))
    lg2 = host(tm.forward(ids[c:], cache))
    assert np.array_equal(np.concatenate([lg1, lg2]), want)
    # every layer of the three passes ran the matrix-core attention, over 2 c, c and 2 c keys
    assert calls == [2 * c] * cfg.NL + [c] * cfg.NL + [2 * c] * cfg.NL
    otoks, orows = O.greedy_decode(om, ids, 4)
    tok = int(lg2[-1].argmax())
    assert tok == otoks[0]
    for i in range(1, 4):
        lgi, nid = tm.decode_rows([tok], cache)
        assert np.array_equal(host(lgi)[0], orows[i]), i
        tok = int(host(nid)[0])


def test_batch_decode_and_graph_replay_match_eager():
    cfg = synth.CONFIGS["tiny"]
    seed = 4
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64, batch=4)
    om = helpers.oracle_model(cfg, seed, T=64)
    prompts = [helpers.prompt(100 + b, 6 + b, cfg.V) for b in range(4)]
    cache = tm.new_cache()
    first = []
    for b, p in enumerate(prompts):
        lg = host(tm.forward(p, cache, slot=b))
        first.append(int(lg[-1].argmax()))
    gd = GraphDecoder(tm, cache, 4)
    gd.load(first)
    gd.capture()
    steps = []
    for _ in range(5):
        lg, ids = gd.step()
        steps.append((host(lg).copy(), host(ids).copy()))
    for b, p in enumerate(prompts):
        otoks, orows = O.greedy_decode(om, p, 6)
        assert otoks[0] == first[b]
        for i in range(5):
            assert np.array_equal(steps[i][0][b], orows[i + 1]), (b, i)
            assert int(steps[i][1][b]) == otoks[i + 1]


@pytest.mark.parametrize("name,T", [("tiny", 12), ("tiny-hd128", 40), ("tiny-hd128", 100)])
def test_graph_prefill_replays_match_oracle(name, T):
    """Prefill captured as a HIP graph (forward(graph=True)): the first call runs eagerly and captures, later calls of
    the same length, slot and start position replay it with new prompts; every replay equals the oracle, with eager
    passes and host synchronisations in between, and a second chunk continues the cache. At hd 128 and 100 rows
    both chunks run the matrix-core attention inside the captured graph; at 40 rows the row kernel."""
    cfg = synth.CONFIGS[name]
    seed = 8
    om = helpers.oracle_model(cfg, seed, T=256)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=256, batch=2)
    cache = tm.new_cache()
    for rep in range(4):
        ids = helpers.prompt(100 + rep, T, cfg.V)
        cache.n[1] = 0
        got = host(tm.forward(ids, cache, slot=1, graph=True))
        assert np.array_equal(got, om(ids)), rep
        more = helpers.prompt(200 + rep, T, cfg.V)
        got2 = host(tm.forward(more, cache, slot=1, graph=True))   # second chunk, start position T
        assert np.array_equal(got2, om(ids + more)[T:]), rep
        # an eager pass on another slot in between
        other = helpers.prompt(300 + rep, 5, cfg.V)
        cache.n[0] = 0
        assert np.array_equal(host(tm.forward(other, cache, slot=0)), om(other))
    assert len(tm._graphs) == 2


def test_slot_outside_the_cache_is_rejected_before_any_launch():
    cfg = synth.CONFIGS["tiny"]
    tm = TModel(DeviceWeights.synthetic(cfg, 2, DEV), Smax=32, batch=2)
    cache = tm.new_cache()
    before = [host(t).copy() for t in cache.layers[0]]
    for bad in (-1, 2, 1.0):
        with pytest.raises(ExactError, match="outside the cache"):
            tm.forward([1, 2, 3], cache, slot=bad)
        with pytest.raises(ExactError, match="outside the cache"):
            tm.forward_traced([1, 2, 3], cache, slot=bad)
    assert all(np.array_equal(host(t), b) for t, b in zip(cache.layers[0], before))
    assert cache.n == [0, 0]


@pytest.mark.parametrize("name,abits,T", [("tiny", 15, 20), ("tiny", 15, 40), ("tiny-moe", 15, 24), ("tiny", 7, 30),
                                          ("tiny-hd128", 15, 100)])
def test_last_only_prefill_matches_full_prefill(name, abits, T):
    """forward(last_only=True) computes the final norm, head and argmax for the last row only: its logits equal the
    full pass's last row, eagerly and as graph replays, and the passes after it on the same workspace (whose residual
    totals the last-row pass must leave cleared) still equal the oracle-pinned full pass."""
    cfg = synth.CONFIGS[name]
    w = DeviceWeights.synthetic(cfg, 5, DEV)
    tm = TModel(w, Smax=2 * T + 8, abits=abits)
    ids = helpers.prompt(11, T, cfg.V)
    full = host(tm.forward(ids, tm.new_cache(B=1)))
    for graph in (False, True, True):
        last = host(tm.forward(ids, tm.new_cache(B=1), last_only=True, graph=graph))
        assert last.shape == (1, cfg.V) and np.array_equal(last[0], full[-1]), graph
    again = host(tm.forward(ids, tm.new_cache(B=1)))
    assert np.array_equal(again, full)
    # a second chunk continuing the cache, last row only, against the same chunk with every row
    c1, c2 = tm.new_cache(B=1), tm.new_cache(B=1)
    tm.forward(ids, c1)
    tm.forward(ids, c2)
    more = helpers.prompt(12, T, cfg.V)
    a = host(tm.forward(more, c1))
    b = host(tm.forward(more, c2, last_only=True))
    assert np.array_equal(b[0], a[-1])
