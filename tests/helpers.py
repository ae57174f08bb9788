"""Shared test helpers: oracle-side models built from the same seeded integers as the device models."""
import numpy as np

import exact_oracle as O
from exact_amd import synth


def lin_np(seed, name, N, K, bias=False):
    kw, km, kb = (synth.key(seed, name + s) for s in (".w", ".m", ".b"))
    w = synth.weights_np(kw, N, K)
    M = synth.scales_np(km, N, K)
    b = synth.vector_np(kb, N, *synth.BIAS) if bias else None
    return w, M, b


def lin_c(seed, name, N, K, bias=False):
    """lin_np through the oracle's C generator (exact_c.c): the same integers, fast enough for 14B."""
    import exact_c
    kw, km, kb = (synth.key(seed, name + s) for s in (".w", ".m", ".b"))
    w = exact_c.weights(kw, synth.thresholds(), N, K)
    M = exact_c.scales(km, N, K, synth.M_LO, synth.M_HI)
    b = synth.vector_np(kb, N, *synth.BIAS) if bias else None
    return w, M, b


def embed_c(ew, eM):
    import exact_c
    return exact_c.embed(ew, eM)


def oracle_weights(cfg, seed, layers=None, lin=lin_np, embed=synth.embed_np):
    """Oracle weights dict (exact_oracle.Model layout) of the synthetic model (seed, cfg)."""
    D, H, KV, hd = cfg.D, cfg.H, cfg.KV, cfg.hd
    nl = cfg.NL if layers is None else layers
    Ls = []
    for li in range(nl):
        L = dict(g1=synth.vector_np(synth.key(seed, f"L{li}.g1"), D, *synth.GAIN),
                 g2=synth.vector_np(synth.key(seed, f"L{li}.g2"), D, *synth.GAIN))
        for name, N, K, bias in synth.linear_specs(cfg, li):
            short = name.split(".", 1)[1]
            L[short] = O.Lin(*lin(seed, name, N, K, bias))
        if cfg.moe:
            L["experts"] = [(L.pop(f"e{e}.gate"), L.pop(f"e{e}.up"), L.pop(f"e{e}.down")) for e in range(cfg.NE)]
        Ls.append(L)
    ew, eM, _ = lin(seed, "emb", cfg.V, D)
    W = dict(layers=Ls, gf=synth.vector_np(synth.key(seed, "gf"), D, *synth.GAIN), emb=embed(ew, eM))
    W["head"] = O.Lin(ew, eM) if cfg.tie else O.Lin(*lin(seed, "head", cfg.V, D))
    return W


def oracle_model(cfg, seed, T=512, layers=None, abits=15, lin=lin_np, embed=synth.embed_np):
    c = dict(D=cfg.D, H=cfg.H, KV=cfg.KV, hd=cfg.hd, NL=cfg.NL if layers is None else layers, theta=cfg.theta, T=T,
             topk=cfg.topk)
    return O.Model(oracle_weights(cfg, seed, layers, lin, embed), c, abits=abits)



def prompt(seed, n, V):
    return np.random.default_rng(seed).integers(0, V, n).tolist()
