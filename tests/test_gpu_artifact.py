"""Models loaded from the on-disk exact artifact (SPEC.md:7-12) on the GPU: group mode equals the oracle and the
device-generated synthetic model; a per-channel artifact of the reference's golden IntModel reproduces the
reference's own logits; the tables used are the artifact's."""
import os

import numpy as np
import pytest
import torch

import exact_oracle as O
import helpers
from exact_amd import artifact, synth, tables
from exact_amd.model import DeviceWeights, TModel

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "intmodel_tiny.npz")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("name", ["tiny", "tiny-tied"])
def test_group_artifact_matches_oracle_and_synthetic(tmp_path, name):
    cfg = synth.CONFIGS[name]
    seed = 12
    artifact.write(str(tmp_path), cfg, synth.arrays(cfg, seed), tables.host_tables(96, cfg.hd, cfg.theta))
    w = DeviceWeights.from_artifact(str(tmp_path), DEV)
    tm = TModel(w, Smax=96)
    assert torch.equal(tm.tab.cos.cpu(), torch.from_numpy(tables.rope(96, cfg.hd, cfg.theta)[0]))
    ids = helpers.prompt(5, 21, cfg.V)
    want = helpers.oracle_model(cfg, seed, T=96)(ids)
    assert np.array_equal(host(tm.forward(ids)), want)
    ts = TModel(DeviceWeights.synthetic(cfg, seed, DEV), Smax=96)
    assert np.array_equal(host(ts.forward(ids)), want)
    # decode through the cache
    cache = tm.new_cache(B=1)
    lg = host(tm.forward(ids[:15], cache))
    tok = int(lg[-1].argmax())
    otoks, orows = O.greedy_decode(helpers.oracle_model(cfg, seed, T=96), ids[:15], 4)
    assert tok == otoks[0]
    for i in range(1, 4):
        lgi, nid = tm.decode_rows([tok], cache)
        assert np.array_equal(host(lgi)[0], orows[i])
        tok = int(host(nid)[0])


def test_channel_artifact_of_the_reference_golden_model(tmp_path):
    z = np.load(GOLD)
    cfg_d = eval(bytes(z["cfg_json"]).decode(), {})
    cfg = synth.ModelConfig("golden", D=cfg_d["D"], H=cfg_d["H"], KV=cfg_d["KV"], hd=cfg_d["hd"], I=cfg_d["I"],
                            V=cfg_d["V"], NL=cfg_d["NL"], theta=cfg_d["theta"])
    arrays = {k: z[k] for k in z.files if k not in ("cfg_json", "prompt", "logits") and not k.startswith("rc_")}
    arrays["emb"] = z["emb"].astype(np.int64)
    artifact.write(str(tmp_path), cfg, arrays, tables.host_tables(cfg_d["T"], cfg.hd, cfg.theta), mode="channel")
    tm = TModel(DeviceWeights.from_artifact(str(tmp_path), DEV), Smax=cfg_d["T"])
    assert np.array_equal(host(tm.forward(z["prompt"].tolist())), z["logits"])
