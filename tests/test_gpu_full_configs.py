"""Full-size models on the GPU against oracle fixtures (tests/golden/make_full_configs.py): every logits
row hash and every greedy token of the Qwen2.5-0.5B, Qwen2.5-7B (the decode benchmark's model, bs1 and bs2),
Qwen2.5-14B (bs1 and bs8) and Qwen1.5-MoE-A2.7B shaped synthetic models. Prefill runs per sequence; decode runs all
sequences as one batch in a HIP graph. The 7B decode runs the path its benchmark times: the attention's residual +
RMSNorm + qrow inside 8-wave q|k|v GEMV blocks, one per CU, and the SwiGLU in the gate|up GEMV's epilogue."""
import json
import os

import numpy as np
import pytest
import torch

import exact_oracle as O
from exact_amd import synth
from exact_amd.model import DeviceWeights, GraphDecoder, TModel

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("name,batch", [("c1", None), ("c2", 1), ("c2", None), ("c5", None), ("c4", 1), ("c4", None)])
def test_full_config_matches_oracle_fixture(name, batch):
    """batch None: every fixture sequence decoded together (bs8 for c4); 1: the first sequence alone."""
    path = os.path.join(GOLD, f"full_{name}.json")
    if not os.path.exists(path):
        pytest.skip(f"{path} not written yet (tests/golden/make_full_configs.py {name})")
    spec = json.load(open(path))
    cfg = synth.CONFIGS[spec["config"]]
    seqs = spec["sequences"] if batch is None else spec["sequences"][:batch]
    B, n = len(seqs), spec["new_tokens"]
    print(f"{name}: {cfg.name} B={B} prompt={spec['prompt_len']} new={n}", flush=True)
    tm = TModel(DeviceWeights.synthetic(cfg, spec["seed"], DEV), Smax=spec["prompt_len"] + n, batch=B,
                abits=spec["abits"])
    cache = tm.new_cache()
    first = []
    for b, sq in enumerate(seqs):
        row = host(tm.forward(sq["prompt"], cache, last_only=True, slot=b))[-1]
        assert O.h(row) == sq["hashes"][0], (b, "prefill")
        first.append(int(row.argmax()))
        assert first[-1] == sq["tokens"][0]
    del tm._ws[spec["prompt_len"]]                      # prefill buffers are not needed for decode
    gd = GraphDecoder(tm, cache, B)
    gd.load(first)
    gd.capture()
    for i in range(1, n):
        lg, nid = gd.step()
        rows, ids = host(lg), host(nid)
        for b, sq in enumerate(seqs):
            assert O.h(rows[b]) == sq["hashes"][i], (b, i)
            assert int(ids[b]) == sq["tokens"][i], (b, i)
