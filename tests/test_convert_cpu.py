"""Float checkpoint -> integer arrays (QLin.__init__, exact_llm.py:83-88; GQLin.__init__, speed_fair_kaggle.py:715-721;
IntModel.__init__, exact_llm.py:141-160). The oracle's quantisers are pinned by closed-form properties; the product
converter must give the oracle's integers, also through a safetensors checkpoint directory."""
import json
import os

import numpy as np
import pytest

import exact_oracle as O
from exact_amd import convert as C


def _props(w_in_out, w8, M, K0=None):
    """Closed-form properties of the per-column quantiser on a float64 (in, out) block."""
    w = np.asarray(w_in_out, np.float64)
    mx = np.abs(w).max(0)
    sc = np.where(mx == 0, 1e-12, mx) / 127.0
    assert np.abs(w8.astype(np.int64)).max() <= 127
    assert M.dtype == np.int64 and np.abs(M - sc * 2.0 ** 28).max() <= 0.5   # the nearest integer to sc 2^28
    for n in range(w.shape[1]):
        if mx[n] == 0:
            assert not w8[:, n].any() and M[n] == 0
            continue
        k = int(np.abs(w[:, n]).argmax())
        assert abs(int(w8[k, n])) == 127 and np.sign(w8[k, n]) == np.sign(w[k, n])
        assert np.abs(w[:, n] - w8[:, n] * sc[n]).max() <= sc[n] / 2 * (1 + 1e-12)


def test_oracle_quantize_channel_closed_form():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.05, (96, 40))
    w[:, 3] = 0.0                                   # an all-zero column
    w[5, 7] = -0.9                                  # the column maximum is negative
    w[:, 9] = 0.25 * np.arange(96) / 95            # a linear ramp: the last element maps to 127
    w8, M = O.quantize_channel(w)
    _props(w, w8, M)
    assert w8[5, 7] == -127 and w8[95, 9] == 127
    # half-way values: w / sc = k + 1/2 rounds to even (numpy rint), as in the reference
    w2 = np.array([[127.0], [0.5], [1.5], [-2.5]])
    w8, M = O.quantize_channel(w2)
    assert w8[:, 0].tolist() == [127, 0, 2, -2] and M[0] == 1 << 28


def test_oracle_quantize_group_is_channel_per_group():
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.03, (384, 24))
    w[128:256, 5] = 0.0
    w8, M = O.quantize_group(w)
    assert M.shape == (3, 24)
    for g in range(3):
        _props(w[g * 128:(g + 1) * 128], w8[g * 128:(g + 1) * 128], M[g])
    assert M[1, 5] == 0 and M[0, 5] > 0


@pytest.mark.parametrize("mode", ["group", "channel"])
def test_product_quantisers_equal_oracle(mode):
    rng = np.random.default_rng(3)
    w_out_in = rng.normal(0, 0.02, (200, 256)).astype(np.float32)   # checkpoint layout (out, in), float32
    if mode == "group":
        a, b = C.quantize_group(w_out_in), O.quantize_group(np.asarray(w_out_in, np.float64).T)
    else:
        a, b = C.quantize_channel(w_out_in), O.quantize_channel(np.asarray(w_out_in, np.float64).T)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def fake_checkpoint(path, D=256, H=4, KV=2, I=384, V=600, NL=2, tie=False, seed=0):
    """A Qwen2-layout float checkpoint with random weights (safetensors + config.json)."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    hd = D // H
    t = {"model.embed_tokens.weight": rng.normal(0, 0.05, (V, D)).astype(np.float32),
         "model.norm.weight": rng.normal(1.0, 0.1, D).astype(np.float32)}
    for i in range(NL):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = rng.normal(1.0, 0.1, D).astype(np.float32)
        t[p + "post_attention_layernorm.weight"] = rng.normal(1.0, 0.1, D).astype(np.float32)
        for nm, (N, K) in {"self_attn.q_proj": (H * hd, D), "self_attn.k_proj": (KV * hd, D), "self_attn.v_proj": (KV * hd, D),
                           "self_attn.o_proj": (D, H * hd), "mlp.gate_proj": (I, D), "mlp.up_proj": (I, D),
                           "mlp.down_proj": (D, I)}.items():
            t[p + nm + ".weight"] = rng.normal(0, 0.04, (N, K)).astype(np.float32)
            if nm in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"):
                t[p + nm + ".bias"] = rng.normal(0, 0.1, N).astype(np.float32)
    if not tie:
        t["lm_head.weight"] = rng.normal(0, 0.05, (V, D)).astype(np.float32)
    os.makedirs(path, exist_ok=True)
    save_file(t, os.path.join(path, "model.safetensors"))
    json.dump(dict(hidden_size=D, num_attention_heads=H, num_key_value_heads=KV, intermediate_size=I, vocab_size=V,
                   num_hidden_layers=NL, rope_theta=1e6, tie_word_embeddings=tie), open(os.path.join(path, "config.json"), "w"))
    return t


def oracle_arrays(t, NL, mode, tie):
    """The same conversion restated with the oracle's quantisers."""
    qz = O.quantize_group if mode == "group" else O.quantize_channel
    out = {"emb": O.q16(t["model.embed_tokens.weight"]), "gf": O.q16(t["model.norm.weight"])}
    for i in range(NL):
        p = f"model.layers.{i}."
        out[f"{i}.g1"] = O.q16(t[p + "input_layernorm.weight"])
        out[f"{i}.g2"] = O.q16(t[p + "post_attention_layernorm.weight"])
        for k, nm in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"), ("o", "self_attn.o_proj"),
                      ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"), ("down", "mlp.down_proj")):
            out[f"{i}.{k}.w"], out[f"{i}.{k}.M"] = qz(np.asarray(t[p + nm + ".weight"], np.float64).T)
            if p + nm + ".bias" in t:
                out[f"{i}.{k}.b"] = O.q16(t[p + nm + ".bias"])
    hw = t["model.embed_tokens.weight"] if tie else t["lm_head.weight"]
    out["head.w"], out["head.M"] = O.quantize_channel(np.asarray(hw, np.float64).T)
    return out


@pytest.mark.parametrize("mode,tie", [("group", False), ("channel", True)])
def test_convert_checkpoint_directory(tmp_path, mode, tie):
    t = fake_checkpoint(str(tmp_path), tie=tie)
    cfg, arr, tab = C.convert_checkpoint(str(tmp_path), mode, T=64)
    assert (cfg.D, cfg.H, cfg.KV, cfg.hd, cfg.I, cfg.V, cfg.NL, cfg.tie) == (256, 4, 2, 64, 384, 600, 2, tie)
    want = oracle_arrays(t, 2, mode, tie)
    assert sorted(arr) == sorted(want)
    for k in want:
        assert np.array_equal(arr[k], want[k]), k
    assert arr["0.q.M"].max() >= 1 << 15          # quantised scales exceed int16: the wide-scale path is needed
    assert tab["cos"].shape == (64, 64)
