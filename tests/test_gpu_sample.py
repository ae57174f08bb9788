"""Device integer sampler and receipts against the oracle (sample_int / generate / verify, exact_llm.py:243-276)."""
import numpy as np
import pytest
import torch

import exact_oracle as O
import helpers
from exact_amd import ops, synth
from exact_amd.model import DeviceWeights, TModel, generate, verify
from exact_amd.tables import exp_t

pytestmark = pytest.mark.gpu
DEV = "cuda"
I32, I64 = torch.int32, torch.int64


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("R,V,temp", [(3, 152064, 1.0), (2, 1000, 0.7), (4, 7, 2.0), (1, 1, 1.0), (2, 5000, 0.05)])
def test_sample_matches_oracle(R, V, temp):
    rng = np.random.default_rng(V + R)
    lg = rng.integers(-(8 << 16), 8 << 16, (R, V))
    if V > 10:
        lg[0, :] = 12345                                # uniform row
        lg[1, V // 3] = 40 << 16                        # one dominant logit: most p are 0
    seed = 0x1234_5678_9ABC_DEF0
    steps = rng.integers(0, 1000, R).astype(np.int32)
    tnum = ops.temp_num(temp)
    ids, pd = torch.zeros(R, dtype=I32, device=DEV), torch.zeros((R, V), dtype=I64, device=DEV)
    ops.sample(torch.tensor(lg, device=DEV), seed, torch.tensor(steps, device=DEV), tnum,
               torch.tensor(exp_t(), dtype=I32, device=DEV), ids, pd)
    got, gp = host(ids), host(pd)
    for r in range(R):
        tok, p = O.sample_int(lg[r], seed, int(steps[r]), tnum)
        assert np.array_equal(gp[r], p), r
        assert got[r] == tok, (r, got[r], tok)


def test_generate_receipt_matches_oracle_and_verifies():
    cfg = synth.CONFIGS["tiny"]
    om = helpers.oracle_model(cfg, 5, T=64)
    tm = TModel(DeviceWeights.synthetic(cfg, 5, DEV), Smax=64)
    prompt = helpers.prompt(8, 7, cfg.V)
    rec, greedy = generate(tm, prompt, 12, seed=99, temp=0.8)
    orec, ogreedy, _ = O.generate(om, prompt, 12, seed=99, temp=0.8)
    assert rec["tokens"] == orec["tokens"] and rec["chain"] == orec["chain"] and greedy == ogreedy
    assert any(a != b for a, b in zip(rec["tokens"], greedy))       # it really samples
    assert verify(tm, rec) == (True, None)
    bad = dict(rec, tokens=list(rec["tokens"]))
    bad["tokens"][5] = (bad["tokens"][5] + 1) % cfg.V
    assert verify(tm, bad) == (False, 5)
    # the host checks each step one step behind the device: the first and last positions and the chain itself
    for pos in (0, 11):
        bad = dict(rec, tokens=list(rec["tokens"]))
        bad["tokens"][pos] = (bad["tokens"][pos] + 1) % cfg.V
        assert verify(tm, bad) == (False, pos)
    assert verify(tm, dict(rec, chain="0" * 16)) == (False, "chain")


@pytest.mark.parametrize("n", [1, 2])
def test_short_generations_match_oracle(n):
    """one token (no decode step) and two (one captured step) through the pipelined receipt path"""
    cfg = synth.CONFIGS["tiny"]
    om = helpers.oracle_model(cfg, 6, T=32)
    tm = TModel(DeviceWeights.synthetic(cfg, 6, DEV), Smax=32)
    prompt = helpers.prompt(3, 5, cfg.V)
    rec, greedy = generate(tm, prompt, n, seed=7, temp=0.9)
    orec, ogreedy, _ = O.generate(om, prompt, n, seed=7, temp=0.9)
    assert rec["tokens"] == orec["tokens"] and rec["chain"] == orec["chain"] and greedy == ogreedy
    assert verify(tm, rec) == (True, None)
