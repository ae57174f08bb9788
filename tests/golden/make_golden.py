"""Writes tests/golden/intmodel_tiny.npz: end-to-end vectors of the reference's numpy IntModel.

The composed forward (IntModel.__call__, exact_llm.py:161-180) and the receipt generator
(generate, exact_llm.py:262-268) are the only parts of the path that no reference-held fixture
pins end to end, so this script imports the reference's exact_llm.py (numpy only, no network) in
the build container, builds a tiny integer model from seeded integers (per-channel QLin objects
created with __new__, so no float quantisation runs), and stores inputs and outputs as data.

Run from the repository root:  python tests/golden/make_golden.py [/path/to/reference]
The reference is needed only to (re)write the fixture; tests read the .npz alone.
"""
import math
import os
import sys

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "intmodel_tiny.npz")

CFG = dict(D=128, H=4, KV=2, hd=32, I=256, V=512, NL=2, T=64, theta=1e4, eps=1e-6, tie=False)


def make_weights(seed=1234):
    c = CFG
    r = np.random.default_rng(seed)
    D, H, KV, hd, I, V = c["D"], c["H"], c["KV"], c["hd"], c["I"], c["V"]

    def lin(K, N, bias):
        w = np.clip(np.rint(r.normal(0, 40, (K, N))), -127, 127).astype(np.int8)
        M = r.integers(1 << 17, 1 << 19, N).astype(np.int64)
        b = r.integers(-(1 << 14), 1 << 14, N).astype(np.int64) if bias else None
        return w, M, b

    W = {"emb": r.integers(-(1 << 13), 1 << 13, (V, D)).astype(np.int64),
         "gf": r.integers(3 << 14, 5 << 14, D).astype(np.int64)}
    for li in range(c["NL"]):
        W[f"{li}.g1"] = r.integers(3 << 14, 5 << 14, D).astype(np.int64)
        W[f"{li}.g2"] = r.integers(3 << 14, 5 << 14, D).astype(np.int64)
        for name, K, N, bias in (("q", D, H * hd, True), ("k", D, KV * hd, True), ("v", D, KV * hd, True),
                                 ("o", H * hd, D, False), ("gate", D, I, False), ("up", D, I, False),
                                 ("down", I, D, False)):
            w, M, b = lin(K, N, bias)
            W[f"{li}.{name}.w"], W[f"{li}.{name}.M"] = w, M
            if b is not None:
                W[f"{li}.{name}.b"] = b
    w, M, _ = lin(D, V, False)
    W["head.w"], W["head.M"] = w, M
    return W


def main():
    sys.path.insert(0, REF)
    import exact_llm as ex                                            # numpy-only module
    W = make_weights()

    def qlin(pfx):
        q = ex.QLin.__new__(ex.QLin)
        q.w = W[pfx + ".w"]
        q.M = W[pfx + ".M"]
        q.Mbits = int(ex.bitlen(np.array([q.M.max()]))[0])
        q.b = W.get(pfx + ".b")
        return q

    c = CFG
    m = ex.IntModel.__new__(ex.IntModel)
    m.c = c
    m.emb = W["emb"].astype(np.float64) / 65536.0                      # rint(emb * 2^16) gives back the integers
    m.layers = [dict(g1=W[f"{i}.g1"], g2=W[f"{i}.g2"], **{k: qlin(f"{i}.{k}") for k in
                                                         ("q", "k", "v", "o", "gate", "up", "down")})
                for i in range(c["NL"])]
    m.gf = W["gf"]
    m.head = qlin("head")
    cos, sin = ex.rope_tables(c["T"], c["hd"], c["theta"])
    m.cos = np.rint(cos * ex.ONE).astype(np.int64)
    m.sin = np.rint(sin * ex.ONE).astype(np.int64)
    prompt = np.random.default_rng(7).integers(0, c["V"], 12).tolist()
    logits = m(prompt)
    receipt, greedy = ex.generate(m, prompt, 6, seed=99, temp=0.8)
    out = {k: (v.astype(np.int16) if k == "emb" else v) for k, v in W.items()}   # emb values fit int16
    out.update(cfg_json=np.frombuffer(repr(CFG).encode(), np.uint8), prompt=np.array(prompt, np.int64),
               logits=logits, logits_hash=np.frombuffer(ex.h(logits).encode(), np.uint8),
               sampled=np.array(receipt["tokens"], np.int64), chain=np.frombuffer(receipt["chain"].encode(), np.uint8),
               greedy=np.array(greedy, np.int64), seed=np.array(99), temp=np.array(0.8),
               inv=np.array(int(round((1 << 16) / math.sqrt(c["hd"])))))
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, "hash", ex.h(logits), "tokens", receipt["tokens"], "greedy", greedy)


if __name__ == "__main__":
    main()
