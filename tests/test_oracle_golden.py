"""Pins the oracle against the reference's own fixtures (webverify/cells_tiny.json)."""
import json
import os

import numpy as np
import pytest

import exact_oracle as O
import cells_replay

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def cells():
    with open(os.path.join(GOLD, "cells_tiny.json")) as f:
        return json.load(f)


def test_tables_match_reference_fixture(cells):
    t = cells["tables"]
    assert t["EXP_STEP"] == O.EXP_STEP and t["SILU_STEP"] == O.SILU_STEP
    assert np.array_equal(np.array(t["EXP_T"], np.int64), O.EXP_T)
    assert np.array_equal(np.array(t["SILU_T"], np.int64), O.SILU_T)
    # spot values quoted from the fixture
    assert list(O.EXP_T[:4]) == [16777216, 16711808, 16646655, 16581756]
    assert list(O.SILU_T[4096:4099]) == [0, 128, 257]


def test_cells_replay_verdicts(cells):
    """Every cell gives the recorded verdict and reason when recomputed with the oracle."""
    for case in cells["cases"]:
        ok, why = cells_replay.replay(case)
        assert ok == case["python_ok"], (case["label"], why)
        assert str(why) == case["python_reason"], (case["label"], why, case["python_reason"])


def test_cells_replay_detects_planted_oracle_mistakes(cells, monkeypatch):
    """A plausible mistake in an oracle primitive makes an honest cell fail (so the replay pins it)."""
    honest = cells["cases"][0]
    assert cells_replay.replay(honest)[0]
    orig_shr = O.round_shift
    orig_softmax = O.isoftmax

    def shr_half_down(a, n):          # round-half-down instead of half-up
        a = np.asarray(a, np.int64)
        n = np.asarray(n, np.int64)
        return np.where(n > 0, (a + (np.left_shift(np.int64(1), np.maximum(n - 1, 0)) - 1)) >> np.maximum(n, 0),
                        a << np.maximum(-n, 0))
    for name, bad in [("round_shift", shr_half_down),
                      ("isilu", lambda x, table=None: O.SILU_T[(np.clip(x, -16 * O.ONE, 16 * O.ONE - 1) + 16 * O.ONE) >> 8]),
                      ("isoftmax", lambda sc, valid, table=None: orig_softmax(sc, valid) + 1),
                      ("rot_half", lambda x: np.concatenate([np.split(x, 2, -1)[1], -np.split(x, 2, -1)[0]], -1))]:
        with monkeypatch.context() as m:
            m.setattr(O, name, bad)
            if name == "round_shift":
                m.setattr(O, "shr", bad)
            assert not cells_replay.replay(honest)[0], name
    assert O.round_shift is orig_shr
