"""A converted float checkpoint on the GPU: group-128 layers with wide (> int16) scales and a per-channel head, as the
reference's group engine builds it (speed_fair_kaggle.py:776-780), and an all-per-channel model (IntModel,
exact_llm.py:141-160): logits and greedy decode equal the oracle model on the oracle's quantisation of the same floats,
also through the on-disk artifact."""
import numpy as np
import pytest
import torch

import exact_oracle as O
from exact_amd import artifact
from exact_amd import convert as C
from exact_amd.model import DeviceWeights, TModel
from test_convert_cpu import fake_checkpoint, oracle_arrays

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def oracle_model(arr, cfg, mode, T):
    layers = []
    for i in range(cfg.NL):
        L = dict(g1=arr[f"{i}.g1"], g2=arr[f"{i}.g2"])
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            L[k] = O.Lin(arr[f"{i}.{k}.w"], arr[f"{i}.{k}.M"], arr.get(f"{i}.{k}.b"), mode=mode)
        layers.append(L)
    W = dict(emb=arr["emb"], gf=arr["gf"], layers=layers, head=O.Lin(arr["head.w"], arr["head.M"], mode="channel"))
    return O.Model(W, dict(D=cfg.D, H=cfg.H, KV=cfg.KV, hd=cfg.hd, NL=cfg.NL, theta=cfg.theta, T=T, topk=0))


@pytest.mark.parametrize("mode,tie", [("group", False), ("channel", True)])
def test_converted_checkpoint_matches_oracle(tmp_path, mode, tie):
    t = fake_checkpoint(str(tmp_path / "ckpt"), tie=tie, seed=4)
    cfg, arr, tab = C.convert_checkpoint(str(tmp_path / "ckpt"), mode, T=64)
    om = oracle_model(oracle_arrays(t, cfg.NL, mode, tie), cfg, mode, 64)
    ids = np.random.default_rng(5).integers(0, cfg.V, 20).tolist()
    want = om(ids)
    tm = TModel(DeviceWeights.from_arrays(cfg, arr, DEV, mode=mode, tables=tab), Smax=64)
    if mode == "group":
        assert tm.w.layers[0]["qkv"].mh is not None and tm.w.head.mode == "channel"
    assert np.array_equal(host(tm.forward(ids)), want)
    # through the artifact, then greedy decode through the cache
    artifact.write(str(tmp_path / "art"), cfg, arr, tab, mode=mode)
    tm2 = TModel(DeviceWeights.from_artifact(str(tmp_path / "art"), DEV), Smax=64)
    assert np.array_equal(host(tm2.forward(ids)), want)
    otoks, orows = O.greedy_decode(om, ids[:12], 5)
    cache = tm2.new_cache(B=1)
    tok = int(host(tm2.forward(ids[:12], cache))[-1].argmax())
    assert tok == otoks[0]
    for i in range(1, 5):
        lg, nid = tm2.decode_rows([tok], cache)
        assert np.array_equal(host(lg)[0], orows[i]), i
        tok = int(host(nid)[0])
