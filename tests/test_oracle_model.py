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


def _permuted_mm(order):
    """exact_mm with the K axis permuted (or reversed) before the float64 product (exact_llm.py:76-79)."""
    base = O.exact_mm

    def mm(a, b):
        K = np.shape(a)[-1]
        p = order(K)
        return base(np.asarray(a)[..., p], np.asarray(b)[p, :])
    return mm


def _permuted_group_acc(order):
    """group_acc with each group's 128 inputs permuted (or reversed)."""
    base = O.group_acc

    def acc(xq, w, G=128):
        p = np.concatenate([g * G + order(G) for g in range(xq.shape[1] // G)])
        return base(np.asarray(xq)[:, p], np.asarray(w)[p, :], G)
    return acc


ORDERS = {"permuted": lambda K: np.random.default_rng(K).permutation(K), "reversed": lambda K: np.arange(K)[::-1]}


@pytest.mark.parametrize("order", sorted(ORDERS))
def test_reduction_order_invariance(golden, order, monkeypatch):
    """The reference's M2/S1 gates: logits hashes are identical under a permuted or reversed reduction order
    (exact_llm.py:76-79, 285-292) for the per-channel golden model, a group-128 model and a MoE model."""
    import helpers
    from exact_amd import synth
    z, cfg, W = golden
    ids = z["prompt"].tolist()
    models = [O.Model(W, cfg)]
    for name in ("tiny", "tiny-moe"):
        models.append(helpers.oracle_model(synth.CONFIGS[name], 5, T=64))
    ref = [O.h(m(ids[:9])) for m in models]
    monkeypatch.setattr(O, "exact_mm", _permuted_mm(ORDERS[order]))
    monkeypatch.setattr(O, "group_acc", _permuted_group_acc(ORDERS[order]))
    assert [O.h(m(ids[:9])) for m in models] == ref
