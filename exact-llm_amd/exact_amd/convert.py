"""Conversion of a float Qwen2-family checkpoint into the exact integer arrays (SPEC.md:7: conversion uses float64
arithmetic; the integer artifact, not the float checkpoint, is what conformance refers to).

Follows the reference's quantisers and model construction:
  per-channel linear  QLin.__init__ (exact_llm.py:83-88), chunked over output rows by qlin_chunked (exact_llm.py:133-139),
                      which gives the same integers since every scale belongs to one output column;
  group-128 linear    GQLin.__init__ (experiments/speed_fair_kaggle.py:715-721);
  model               IntModel.__init__ (exact_llm.py:141-160): Q16 norm gains and biases, layers per-channel or
                      (the group engine, speed_fair_kaggle.py:776-780) group-128, the head per-channel from the
                      embedding (tied) or lm_head; embedding rows as Q16 integers, as the lookup at exact_llm.py:163
                      makes them;
  checkpoint access   open_hf (exact_llm.py:213-231) without the download: a local directory of *.safetensors files
                      and config.json.
The result feeds DeviceWeights.from_arrays or artifact.write.
"""
import glob
import json
import os

import numpy as np

from ._lib import ExactError
from .synth import ModelConfig

ONE = 1 << 16
PFX = "model.layers.{}."
LINEARS = (("q", "self_attn.q_proj", True), ("k", "self_attn.k_proj", True), ("v", "self_attn.v_proj", True),
           ("o", "self_attn.o_proj", False), ("gate", "mlp.gate_proj", False), ("up", "mlp.up_proj", False),
           ("down", "mlp.down_proj", False))


def q16(v):
    """rint(v * 2^16) as int64, from float64."""
    return np.rint(np.asarray(v, np.float64) * ONE).astype(np.int64)


def _scale(w):
    """Column scales max|w| / 127 (an all-zero column takes 1e-12 / 127) of a float64 block."""
    sc = np.abs(w).max(0)
    return np.where(sc == 0, 1e-12, sc) / 127.0


def quantize_channel(w_out_in):
    """(w8 (K, N) int8, M (N,) int64) of a checkpoint weight in its (out, in) layout."""
    w = np.asarray(w_out_in, np.float64).T
    sc = _scale(w)
    return np.clip(np.rint(w / sc), -127, 127).astype(np.int8), np.rint(sc * (1 << 28)).astype(np.int64)


def quantize_group(w_out_in, G=128):
    """(w8 (K, N) int8, M (K/G, N) int64): the per-channel rule per G-row group of the (in, out) weight."""
    w = np.asarray(w_out_in, np.float64).T
    K, N = w.shape
    if K % G:
        raise ExactError(f"group-{G} quantisation needs K % {G} == 0 (K = {K})")
    w8 = np.empty((K, N), np.int8)
    M = np.empty((K // G, N), np.int64)
    for gi in range(K // G):
        blk = w[gi * G:(gi + 1) * G]
        sc = _scale(blk)
        w8[gi * G:(gi + 1) * G] = np.clip(np.rint(blk / sc), -127, 127).astype(np.int8)
        M[gi] = np.rint(sc * (1 << 28)).astype(np.int64)
    return w8, M


def config_from_hf(cf, name="checkpoint"):
    """ModelConfig of a Qwen2 config.json dict (open_hf, exact_llm.py:228-231)."""
    theta = cf.get("rope_theta") or (cf.get("rope_parameters") or {}).get("rope_theta", 1e6)
    return ModelConfig(name, D=cf["hidden_size"], H=cf["num_attention_heads"], KV=cf["num_key_value_heads"],
                       hd=cf["hidden_size"] // cf["num_attention_heads"], I=cf["intermediate_size"], V=cf["vocab_size"],
                       NL=cf["num_hidden_layers"], theta=float(theta), tie=bool(cf.get("tie_word_embeddings", False)))


def open_safetensors(path):
    """(get(name) -> float array, config dict) of a local checkpoint directory (*.safetensors + config.json)."""
    from safetensors import safe_open
    files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise ExactError(f"no *.safetensors files in {path}")
    index = {}
    for f in files:
        with safe_open(f, "np") as fh:
            for k in fh.keys():
                index[k] = f

    def get(k):
        if k not in index:
            raise KeyError(k)
        with safe_open(index[k], "np") as fh:
            return fh.get_tensor(k)

    with open(os.path.join(path, "config.json")) as f:
        cf = json.load(f)
    cf.setdefault("tie_word_embeddings", "lm_head.weight" not in index)
    get.names = set(index)
    return get, cf


def convert(get, cfg, mode="group"):
    """Integer arrays (DeviceWeights.from_arrays layout) of a float checkpoint: layers in `mode` ('group' or
    'channel'), the head per-channel (as the reference's engines keep it)."""
    if mode not in ("group", "channel"):
        raise ExactError(f"linear mode {mode!r}")
    quant = quantize_group if mode == "group" else quantize_channel
    names = getattr(get, "names", None)
    out = {}
    emb = np.asarray(get("model.embed_tokens.weight"))
    out["emb"] = q16(emb)
    for i in range(cfg.NL):
        p = PFX.format(i)
        out[f"{i}.g1"] = q16(get(p + "input_layernorm.weight"))
        out[f"{i}.g2"] = q16(get(p + "post_attention_layernorm.weight"))
        for key, nm, bias in LINEARS:
            out[f"{i}.{key}.w"], out[f"{i}.{key}.M"] = quant(get(p + nm + ".weight"))
            if bias and (names is None or p + nm + ".bias" in names):
                out[f"{i}.{key}.b"] = q16(get(p + nm + ".bias"))
    out["gf"] = q16(get("model.norm.weight"))
    out["head.w"], out["head.M"] = quantize_channel(emb if cfg.tie else get("lm_head.weight"))
    return out


def convert_checkpoint(path, mode="group", T=4096):
    """(cfg, arrays, tables) of a local checkpoint directory; RoPE tables for T positions."""
    from .tables import host_tables
    get, cf = open_safetensors(path)
    cfg = config_from_hf(cf, os.path.basename(os.path.normpath(path)))
    return cfg, convert(get, cfg, mode), host_tables(T, cfg.hd, cfg.theta)
