"""Pins the oracle's MoE block and integer sigmoid to vectors of the reference's own code.

tests/golden/moe_tiny.npz was written by tests/golden/make_golden_moe.py, which ran the reference's
MoEInt.moe (experiments/moe_exact_kaggle.py:454-467), SIG_T / isig (:419-424) and GQLin
(experiments/speed_fair_kaggle.py:713-725) on tiny seeded integer layers: one with per-channel linears, one
with group-128 linears, router columns equal in pairs and triples so that probabilities tie across the
top-k boundary. Plausible mistakes planted in the oracle must change the result.
"""
import os

import numpy as np
import pytest

import exact_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "moe_tiny.npz")
MODES = ("channel", "group")


@pytest.fixture(scope="module")
def z():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def layer(z, mode):
    NE = int(z["cfg"][0])

    def lin(name):
        return O.Lin(z[f"{mode}.{name}.w"], z[f"{mode}.{name}.M"].astype(np.int64), mode=mode)
    L = {k: lin(k) for k in ("router", "sgate", "sg", "su", "sd")}
    L["experts"] = [tuple(lin(f"ex{e}.{p}") for p in ("gate", "up", "down")) for e in range(NE)]
    return L


def model(z):
    NE, topk = int(z["cfg"][0]), int(z["cfg"][1])
    return O.Model(dict(layers=[]), dict(D=0, H=1, KV=1, hd=2, NL=0, theta=1e4, T=1, topk=topk, NE=NE))


def run(z, mode):
    stats = []
    y = model(z).moe(layer(z, mode), z[f"{mode}.m"], stats)
    return y, stats[0]


def test_sig_table_and_isig_match_reference(z):
    assert np.array_equal(O.SIG_T, z["SIG_T"])
    assert np.array_equal(O.isig(z["isig_x"]), z["isig_y"])


@pytest.mark.parametrize("mode", MODES)
def test_router_probabilities_and_selection(z, mode):
    L = layer(z, mode)
    m = z[f"{mode}.m"]
    p = O.isoftmax(L["router"](m), np.ones((m.shape[0], int(z["cfg"][0])), bool))
    assert np.array_equal(p, z[f"{mode}.p"])
    assert np.array_equal(O.moe_route(p, int(z["cfg"][1])), z[f"{mode}.sel"])


@pytest.mark.parametrize("mode", MODES)
def test_moe_block_matches_reference(z, mode):
    y, sel = run(z, mode)
    assert np.array_equal(sel, z[f"{mode}.sel"])
    assert np.array_equal(y, z[f"{mode}.y"])
    assert O.h(y) == z[f"{mode}.hash"].tobytes().decode()


def test_fixture_has_boundary_ties(z):
    """The top-k boundary falls inside a tie in some rows, so the tie rule decides expert membership."""
    for mode in MODES:
        p, sel = z[f"{mode}.p"], z[f"{mode}.sel"]
        k = int(z["cfg"][1])
        kth = np.take_along_axis(p, sel[:, k - 1:k], 1)[:, 0]
        nxt = np.sort(p, 1)[:, ::-1][:, k]
        assert (kth == nxt).sum() >= 4


def _renormalised(p, sel, rows, e, ye):          # weights renormalised over the selected experts
    tot = np.take_along_axis(p, sel, 1).sum(1)
    w = (p[rows, e] << 20) // tot[rows]
    return O.round_shift(w[:, None] * ye, 20)


def _shift16(p, sel, rows, e, ye):                # Q20 weight taken as Q16
    return O.round_shift(p[rows, e][:, None] * ye, 16)


def _ties_high(p, k):                             # equal probabilities to the higher expert index
    NE = p.shape[1]
    return NE - 1 - np.argsort(-p[:, ::-1], axis=-1, kind="stable")[:, :k]


def _sig_step(x, table=None):                     # table lookup without the linear interpolation
    x = np.asarray(x, np.int64)
    y = O.SIG_T[(np.clip(x, -16 * O.ONE, 16 * O.ONE - 1) + 16 * O.ONE) >> 8]
    return np.where(x >= 16 * O.ONE, O.ONE, np.where(x < -16 * O.ONE, 0, y))


@pytest.mark.parametrize("name,bad", [("moe_weighted", _renormalised), ("moe_weighted", _shift16),
                                      ("moe_route", _ties_high)])
@pytest.mark.parametrize("mode", MODES)
def test_planted_mistakes_fail(z, mode, name, bad, monkeypatch):
    monkeypatch.setattr(O, name, bad)
    y, sel = run(z, mode)
    assert not (np.array_equal(y, z[f"{mode}.y"]) and np.array_equal(sel, z[f"{mode}.sel"]))


def test_planted_sigmoid_mistake_fails(z, monkeypatch):
    monkeypatch.setattr(O, "isig", _sig_step)
    assert not np.array_equal(O.isig(z["isig_x"]), z["isig_y"])
