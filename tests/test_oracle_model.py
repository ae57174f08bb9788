"""Oracle model composition vs the reference IntModel golden vectors, plus KV-cache invariants."""
import os

import numpy as np
import pytest

import exact_oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "intmodel_tiny.npz")


def load_golden():
    z = np.load(GOLD)
    cfg = eval(bytes(z["cfg_json"]).decode(), {})
    NL = cfg["NL"]
    layers = []
    for i in range(NL):
        L = dict(g1=z[f"{i}.g1"], g2=z[f"{i}.g2"])
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            b = z[f"{i}.{k}.b"] if f"{i}.{k}.b" in z else None
            L[k] = O.Lin(z[f"{i}.{k}.w"], z[f"{i}.{k}.M"], b, mode="channel")
        layers.append(L)
    W = dict(emb=z["emb"].astype(np.int64), layers=layers, gf=z["gf"],
             head=O.Lin(z["head.w"], z["head.M"], None, mode="channel"))
    return z, cfg, W


@pytest.fixture(scope="module")
def golden():
    return load_golden()


def test_forward_matches_reference_intmodel(golden):
    z, cfg, W = golden
    m = O.Model(W, cfg)
    lg = m(z["prompt"].tolist())
    assert np.array_equal(lg, z["logits"])
    assert O.h(lg) == bytes(z["logits_hash"]).decode()


def test_generate_receipt_matches_reference(golden):
    z, cfg, W = golden
    m = O.Model(W, cfg)
    for cached in (False, True):
        rec, gr, _ = O.generate(m, z["prompt"].tolist(), len(z["sampled"]), seed=int(z["seed"]),
                                temp=float(z["temp"]), cached=cached)
        assert rec["tokens"] == z["sampled"].tolist()
        assert gr == z["greedy"].tolist()
        assert rec["chain"] == bytes(z["chain"]).decode()


def test_kv_cache_equals_full_recompute(golden):
    """attention_tc_longctx_kaggle.py:641-643: prefix in one call, then one token at a time."""
    z, cfg, W = golden
    m = O.Model(W, cfg)
    ids = np.random.default_rng(3).integers(0, cfg["V"], 20).tolist()
    full = m(ids)
    cache = m.new_cache()
    part = m(ids[:13], cache)
    assert np.array_equal(part, full[:13])
    for i in range(13, 20):
        assert np.array_equal(m([ids[i]], cache)[0], full[i])


def test_planted_layer_order_mistake_is_caught(golden):
    """Swapping gate and up (a plausible misreading) changes the golden logits."""
    z, cfg, W = golden
    W2 = dict(W)
    W2["layers"] = [dict(L, gate=L["up"], up=L["gate"]) for L in W["layers"]]
    assert not np.array_equal(O.Model(W2, cfg)(z["prompt"].tolist()), z["logits"])
