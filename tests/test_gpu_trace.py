"""Trace capture on the GPU (experiments/gpu_engine_trace_verify_kaggle.py:776-857,
experiments/prover_commit_cost_gpu_kaggle.py:791-845): the totals t of every linear, captured in a prefill
pass and in graph-replayed decode steps, equal the oracle's, pass the Freivalds check with inputs replayed by
the oracle, and leave the logits unchanged; single-entry tampers are rejected."""
import numpy as np
import pytest
import torch

import exact_oracle as O
import helpers
from exact_amd import synth
from exact_amd import trace as TR
import trace_verifier as TV
from exact_amd.model import DeviceWeights, GraphDecoder, TModel

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("q", "k", "v", "o", "gate", "up", "down")


class Recording(O.Model):
    """The oracle model, recording (xq, t) of every linear call under the reference's trace names."""

    def __init__(self, base):
        self.__dict__.update(base.__dict__)
        self.names = {id(L[n]): f"L{i}.{n}" for i, L in enumerate(self.w["layers"]) for n in NAMES}
        self.names[id(self.w["head"])] = "head"
        self.rec = []

    def lin(self, L, x):
        y, t = O.linear_group_t(x, L.w, L.M, L.b, self.abits)
        self.rec.append((self.names[id(L)], O.qrow(np.asarray(x, np.int64), self.abits)[0], t))
        return y

    def take(self):
        out, self.rec = {n: (xq, t) for n, xq, t in self.rec}, []
        return out


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("name,T", [("tiny", 20), ("tiny-hd128", 40)])
def test_prefill_trace_equals_oracle_totals(name, T):
    cfg = synth.CONFIGS[name]
    seed = 5
    om = Recording(helpers.oracle_model(cfg, seed, T=64))
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64)
    ids = helpers.prompt(3, T, cfg.V)
    lg, tr = tm.forward_traced(ids)
    want = om(ids)
    rec = om.take()
    assert np.array_equal(host(lg), want)
    assert np.array_equal(host(tm.forward(ids)), want)          # the untraced pass gives the same logits
    assert sorted(tr) == sorted(rec)
    for n, (_, t) in rec.items():
        assert np.array_equal(tr[n], t), n


def test_freivalds_verifies_the_gpu_trace_and_rejects_tampers():
    """V1/V2 of the reference's trace-verify gates on a synthetic model: every traced linear of a 24-token
    prefill passes with the oracle's replayed inputs; 20 single +-1 changes are each rejected."""
    cfg = synth.CONFIGS["tiny"]
    seed = 6
    base = helpers.oracle_model(cfg, seed, T=64)
    om = Recording(base)
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64)
    ids = helpers.prompt(4, 24, cfg.V)
    _, tr = tm.forward_traced(ids)
    om(ids)
    rec = om.take()
    rng = np.random.default_rng(2026)
    lins = {f"L{i}.{n}": L[n] for i, L in enumerate(base.w["layers"]) for n in NAMES}
    lins["head"] = base.w["head"]
    keys = {n: TV.freivalds_keys(L.w, L.M, rng) for n, L in lins.items()}
    for n in lins:
        assert TV.freivalds_check(keys[n], rec[n][0], tr[n]), n
    names = sorted(lins)
    for i in range(20):
        n = names[rng.integers(len(names))]
        bad = tr[n].copy()
        bad[rng.integers(bad.shape[0]), rng.integers(bad.shape[1])] += 1 if i % 2 else -1
        assert not TV.freivalds_check(keys[n], rec[n][0], bad), n


def test_graph_decode_trace_commitment_and_logits():
    """Decode steps replayed from the two trace graphs: logits equal the untraced graph's, each step's trace
    (copied to pinned memory on a side stream) equals the oracle's totals for that step, and each digest is
    the commitment of that trace."""
    cfg = synth.CONFIGS["tiny"]
    seed = 7
    om = Recording(helpers.oracle_model(cfg, seed, T=64))
    tm = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=64, batch=1)
    ids = helpers.prompt(8, 10, cfg.V)
    steps = 5
    runs = {}
    for trace in (False, True):
        cache = tm.new_cache(B=1)
        lg = tm.forward(ids, cache, last_only=True)
        gd = GraphDecoder(tm, cache, 1, trace=trace)
        gd.load([int(host(lg)[0].argmax())])
        gd.capture()
        rec = gd.record("commit", keep=True) if trace else None
        rows = []
        for _ in range(steps):
            lgs, _ = gd.step()
            rows.append(host(lgs)[0].copy())
        runs[trace] = (rows, rec.finish() if rec else None, rec.kept if rec else None, gd)
    rows0, _, _, _ = runs[False]
    rows1, digests, kept, gd = runs[True]
    assert all(np.array_equal(a, b) for a, b in zip(rows0, rows1))
    assert len(digests) == steps and len(kept) == steps
    # oracle: prefill, then the same greedy tokens one at a time through its cache
    ocache = om.new_cache()
    olg = om(ids, ocache)
    om.take()
    tok = int(olg[-1].argmax())
    for j in range(steps):
        olg = om([tok], ocache)
        rec = om.take()
        assert np.array_equal(olg[0], rows1[j]), j
        got = gd.layout.split(kept[j])
        for n, (_, t) in rec.items():
            assert np.array_equal(got[n], t), (j, n)
        assert digests[j] == TR.commit(kept[j])
        tok = int(olg[0].argmax())
