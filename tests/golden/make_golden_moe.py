"""Writes tests/golden/moe_tiny.npz: vectors of the reference's own MoE block and integer sigmoid.

The MoE block (MoEInt.moe, experiments/moe_exact_kaggle.py:454-467), its integer sigmoid
(SIG_T / isig, :419-424) and the group-128 linear (GQLin, experiments/speed_fair_kaggle.py:713-725) exist
only inside experiment scripts whose top level downloads a checkpoint, so they are never run as scripts.
In the build container this script imports the reference's numpy exact_llm.py (the MoE script's lines
14-125 are the same primitives, byte for byte), takes the text of those three definitions from the two
files, executes only that text in exact_llm's namespace, and calls the MoE block on tiny seeded integer
layers. It stores inputs and outputs as data; the tests read the .npz alone.

Two layers are written: per-channel linears (QLin, as the MoE experiment quantises them) and group-128
linears (GQLin, the mode of the 60-expert configuration). Router columns are made equal in triples so
that probabilities tie, also across the top-k boundary, and the lower expert index must win.

Run from the repository root:  python tests/golden/make_golden_moe.py [/path/to/reference]
"""
import os
import sys
import textwrap

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "moe_tiny.npz")

NE, TOPK, MI, SI, T = 6, 4, 128, 128, 24
DIM = {"channel": 128, "group": 256}   # model width per layer mode (two groups of 128 in the group-128 layer)
# experts whose router columns are equal (so their probabilities tie in every row)
TIES = ((1, 4), (2, 3, 5))   # expert 0 has its own column


def span(path, first, last_pred):
    """Text of the definition that starts at the line `first` matches and runs while last_pred(line) holds."""
    lines = open(path).read().split("\n")
    i = next(k for k, ln in enumerate(lines) if ln.startswith(first))
    j = i + 1
    while j < len(lines) and last_pred(lines[j]):
        j += 1
    return "\n".join(lines[i:j]), i + 1, j


def load_reference():
    sys.path.insert(0, REF)
    import exact_llm as ex                                              # numpy-only module
    moe_py = os.path.join(REF, "experiments", "moe_exact_kaggle.py")
    fair_py = os.path.join(REF, "experiments", "speed_fair_kaggle.py")
    sig, a, b = span(moe_py, "SIG_T = np.array(", lambda ln: ln.startswith(("def isig", "    ")))
    assert (a, b) == (419, 424), (a, b)
    moe, a, b = span(moe_py, "    def moe(s, L, m, stats=None):", lambda ln: ln.startswith("        "))
    assert (a, b) == (454, 467), (a, b)
    gq, a, b = span(fair_py, "G_ = 128", lambda ln: ln.startswith(("class GQLin", "    ")))
    assert (a, b) == (713, 725), (a, b)
    ns = dict(vars(ex))
    ns.update(NE=NE, TOPK=TOPK)
    exec(compile(sig, moe_py, "exec"), ns)
    exec(compile(textwrap.dedent(moe), moe_py, "exec"), ns)
    exec(compile(gq, fair_py, "exec"), ns)
    return ex, ns


def make_layer(r, mode, D):
    """Seeded integer linears: w int8 (K, N) from a clipped N(0, 40^2); channel M (N,) or group M (K/128, N)."""
    def lin(K, N, cols=None):
        w = np.clip(np.rint(r.normal(0, 40, (K, N))), -127, 127).astype(np.int8)
        M = (r.integers(1 << 17, 1 << 19, N) if mode == "channel" else r.integers(1 << 12, 1 << 15, (K // 128, N)))
        M = np.asarray(M, np.int64)
        for grp in cols or ():
            for e in grp[1:]:
                w[:, e] = w[:, grp[0]]
                M[..., e] = M[..., grp[0]]
        return dict(w=w, M=M)
    L = dict(router=lin(D, NE, TIES), sgate=lin(D, 1), sg=lin(D, SI), su=lin(D, SI), sd=lin(SI, D))
    for e in range(NE):
        L[f"ex{e}.gate"], L[f"ex{e}.up"], L[f"ex{e}.down"] = lin(D, MI), lin(D, MI), lin(MI, D)
    return L


def ref_linear(ex, ns, arrs, mode):
    if mode == "channel":
        q = ex.QLin.__new__(ex.QLin)
        q.w, q.M = arrs["w"], arrs["M"]
        q.Mbits = int(ex.bitlen(np.array([q.M.max()]))[0])
        q.b = None
        return q
    q = ns["GQLin"].__new__(ns["GQLin"])
    q.w, q.M, q.b = arrs["w"], arrs["M"], None
    q.groups = [(a, a + 128) for a in range(0, arrs["w"].shape[0], 128)]
    return q


def main():
    ex, ns = load_reference()
    out = dict(cfg=np.array([NE, TOPK, MI, SI, T]), SIG_T=ns["SIG_T"])
    x = np.arange(-20 * ex.ONE, 20 * ex.ONE, 997, dtype=np.int64)        # isig over its table and both clamps
    out["isig_x"], out["isig_y"] = x, ns["isig"](x)
    for li, mode in enumerate(("channel", "group")):
        r = np.random.default_rng(2024 + li)
        D = DIM[mode]
        Ls = make_layer(r, mode, D)
        L = {k: ref_linear(ex, ns, Ls[k], mode) for k in ("router", "sgate", "sg", "su", "sd")}
        L["ex"] = [tuple(ref_linear(ex, ns, Ls[f"ex{e}.{p}"], mode) for p in ("gate", "up", "down")) for e in range(NE)]
        m = r.integers(-3 * ex.ONE, 3 * ex.ONE, (T, D)).astype(np.int64)
        m[0] = 0                                                        # an all-zero row
        m[1, :] = 5 * ex.ONE                                            # a constant row
        stats = []
        y = ns["moe"](None, L, m, stats)
        p = ex.isoftmax(L["router"](m), np.ones((T, NE), bool))
        for k, v in Ls.items():
            out[f"{mode}.{k}.w"], out[f"{mode}.{k}.M"] = v["w"], v["M"].astype(np.int32)
        out[f"{mode}.m"], out[f"{mode}.y"] = m, y
        out[f"{mode}.p"], out[f"{mode}.sel"] = p, stats[0]
        out[f"{mode}.hash"] = np.frombuffer(ex.h(y).encode(), np.uint8)
        # rows whose top-k boundary falls inside a tie (the tie rule decides membership, not only order)
        kth, nxt = np.take_along_axis(p, stats[0][:, TOPK - 1:TOPK], 1), np.sort(p, 1)[:, ::-1][:, TOPK:TOPK + 1]
        print(mode, "hash", ex.h(y), "rows with a tie across the top-k boundary:", int((kth == nxt).sum()))
    np.savez_compressed(OUT, **out)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
