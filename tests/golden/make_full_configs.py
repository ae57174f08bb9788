"""Expected outputs of the full-size configurations, computed by the oracle on the CPU.

    python tests/golden/make_full_configs.py c1|c4|c5 [...]

Each run builds the seeded synthetic model (the same integers exact_amd.synth.weights_np would give,
through the oracle's C generator), runs the oracle with its C group-128 linear, and writes
tests/golden/full_<name>.json: the prompts, the greedy tokens, and the conformance hash (sha256 of the
int64 row, first 16 hex digits; exact_llm.py:22) of every logits row that produced a token.

  c1  Qwen2.5-0.5B shape, 16-token prompt, 64 greedy tokens, bs1
  c2  Qwen2.5-7B shape (the decode benchmark's model: the same seed), 16-token prompt, 24 greedy tokens, bs1 and bs2
  c4  Qwen2.5-14B shape, 128-token prompt, 48 greedy tokens, bs1 and bs8 (8 prompts)
  c5  Qwen1.5-MoE-A2.7B shape, 256-token prompt, 32 greedy tokens, bs1
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "exact-llm_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    sys.path.insert(0, p)

import exact_c  # noqa: E402
import exact_oracle as O  # noqa: E402
import helpers  # noqa: E402
from exact_amd import synth  # noqa: E402

RUNS = {
    "c1": dict(cfg="qwen2.5-0.5b", seed=101, prompt=16, new=64, batch=1),
    "c2": dict(cfg="qwen2.5-7b", seed=11, prompt=16, new=24, batch=2),
    "c4": dict(cfg="qwen2.5-14b", seed=104, prompt=128, new=48, batch=8),
    "c5": dict(cfg="qwen1.5-moe-a2.7b", seed=105, prompt=256, new=32, batch=1),
}


def run(name):
    spec = RUNS[name]
    cfg = synth.CONFIGS[spec["cfg"]]
    t0 = time.time()
    exact_c.install()
    T = spec["prompt"] + spec["new"]
    om = helpers.oracle_model(cfg, spec["seed"], T=T, lin=helpers.lin_c, embed=helpers.embed_c)
    print(f"{name}: weights in {time.time() - t0:.0f} s", flush=True)
    prompts = [helpers.prompt(spec["seed"] * 1000 + b, spec["prompt"], cfg.V) for b in range(spec["batch"])]
    seqs = []
    for b, p in enumerate(prompts):
        t1 = time.time()
        toks, rows = O.greedy_decode(om, p, spec["new"])
        seqs.append(dict(prompt=p, tokens=[int(t) for t in toks], hashes=[O.h(r) for r in rows]))
        print(f"{name}: sequence {b} in {time.time() - t1:.0f} s, tokens {toks[:8]}...", flush=True)
    out = dict(config=spec["cfg"], seed=spec["seed"], abits=15, prompt_len=spec["prompt"], new_tokens=spec["new"],
               sequences=seqs)
    with open(os.path.join(HERE, f"full_{name}.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"{name}: done in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    for n in sys.argv[1:]:
        run(n)
