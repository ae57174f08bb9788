"""Seeded synthetic integer models (the artifact of SPEC.md:7-12, generated instead of downloaded).

The reference only builds integer models by quantising downloaded float checkpoints
(exact_llm.py:82-88, 213-231), which cannot run offline. A synthetic model here is a pure function
of (seed, tensor name, element index):

  u(key, i)   = splitmix64(key, i) >> 32                     (32-bit uniform, counter based)
  W[n][k]     = -127 + #{j : thr[j] <= u(key_w, n*K + k)}     thr = 254 thresholds of round(clip(N(0, 40^2)))
  M[g][n]     = lo + ((u(key_m, n*G + g) * (hi - lo)) >> 32) positive group-128 scale, int16
  vectors     = lo + ((u(key, i) * (hi - lo)) >> 32)          gains (Q16 ~ 1.0), biases (Q16)
  embedding   = Q16 rows rint(E[v][k] * M_E[k/128][v] / 2^12) of an int8 table E (tied: E is the head)

The same function runs in numpy (for the oracle side of a test) and as a HIP kernel (for the device
model), so a multi-GB model is generated on the GPU in milliseconds and any tensor can be regenerated
on the host bit-for-bit.
"""
import functools
import hashlib
import math
from dataclasses import dataclass

import numpy as np

GOLD = np.uint64(0x9E3779B97F4A7C15)
M_LO, M_HI = 8192, 24576          # int16 group scales
GAIN = (3 << 14, 5 << 14)         # Q16 gains in [0.75, 1.25)
BIAS = (-(1 << 14), 1 << 14)      # Q16 biases in [-0.25, 0.25)


@dataclass(frozen=True)
class ModelConfig:
    name: str
    D: int
    H: int
    KV: int
    hd: int
    I: int
    V: int
    NL: int
    theta: float = 1e6
    tie: bool = False
    NE: int = 0        # routed experts (0: dense model)
    topk: int = 0
    MI: int = 0        # expert intermediate
    SI: int = 0        # shared expert intermediate

    @property
    def moe(self):
        return self.NE > 0


CONFIGS = {
    # Qwen2.5-0.5B architecture (tied head)
    "qwen2.5-0.5b": ModelConfig("qwen2.5-0.5b", D=896, H=14, KV=2, hd=64, I=4864, V=151936, NL=24, tie=True),
    # Qwen2.5-7B architecture
    "qwen2.5-7b": ModelConfig("qwen2.5-7b", D=3584, H=28, KV=4, hd=128, I=18944, V=152064, NL=28),
    # Qwen2.5-14B architecture
    "qwen2.5-14b": ModelConfig("qwen2.5-14b", D=5120, H=40, KV=8, hd=128, I=13824, V=152064, NL=48),
    # Qwen1.5-MoE-A2.7B architecture: 60 routed experts top-4, shared expert 5632
    "qwen1.5-moe-a2.7b": ModelConfig("qwen1.5-moe-a2.7b", D=2048, H=16, KV=16, hd=128, I=0, V=151936, NL=24,
                                     NE=60, topk=4, MI=1408, SI=5632),
    # small models for tests
    "tiny": ModelConfig("tiny", D=256, H=4, KV=2, hd=64, I=384, V=1000, NL=2, theta=1e4),
    "tiny-tied": ModelConfig("tiny-tied", D=128, H=2, KV=1, hd=64, I=256, V=700, NL=2, tie=True),
    "tiny-hd128": ModelConfig("tiny-hd128", D=256, H=2, KV=1, hd=128, I=384, V=900, NL=2, theta=1e4),
    "tiny-moe": ModelConfig("tiny-moe", D=256, H=4, KV=4, hd=64, I=0, V=800, NL=2, NE=6, topk=2, MI=128, SI=256),
}


# ----------------------------------------------------------------------------- keys and uniforms
def _fnv1a64(s):
    h = 0xCBF29CE484222325
    for b in s.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _mix64(z):
    z &= 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
    return z ^ (z >> 31)


def key(seed, name):
    """64-bit stream key of tensor `name` in the model of `seed`."""
    return _mix64((seed * 0x9E3779B97F4A7C15) ^ _fnv1a64(name))


def splitmix64_np(k, idx):
    """splitmix64(key, i) for a uint64 index array (numpy wraps uint64 arithmetic)."""
    z = np.uint64(k) + (idx.astype(np.uint64) + np.uint64(1)) * GOLD
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def u32_np(k, idx):
    return splitmix64_np(k, idx) >> np.uint64(32)


@functools.lru_cache(None)
def thresholds():
    """254 uint32 thresholds: thr[j] = round(2^32 * Phi((j - 126.5) / 40)), so that
    w = -127 + #{j : thr[j] <= u} has the law of clip(rint(N(0, 40^2)), -127, 127) to 2^-32."""
    out = []
    for j in range(254):
        z = (j - 127 + 0.5) / 40.0
        p = 0.5 * math.erfc(-z / math.sqrt(2.0))
        out.append(min(int(round(p * 2 ** 32)), 2 ** 32 - 1))
    return np.array(out, np.uint32)


def weights_np(k, N, K, n0=0, n1=None):
    """W (K, N1-N0) int8 for output rows [n0, n1) of an (N out, K in) synthetic matrix."""
    n1 = N if n1 is None else n1
    n = np.arange(n0, n1, dtype=np.uint64)[None, :]
    kk = np.arange(K, dtype=np.uint64)[:, None]
    u = u32_np(k, n * np.uint64(K) + kk)
    return (np.searchsorted(thresholds(), u.astype(np.uint32), side="right") - 127).astype(np.int8)


def scales_np(k, N, K, lo=M_LO, hi=M_HI):
    """M (G, N) int64 group-128 scales."""
    G = K // 128
    n = np.arange(N, dtype=np.uint64)[None, :]
    g = np.arange(G, dtype=np.uint64)[:, None]
    u = u32_np(k, n * np.uint64(G) + g)
    return (lo + ((u * np.uint64(hi - lo)) >> np.uint64(32)).astype(np.int64)).astype(np.int64)


def vector_np(k, n, lo, hi):
    u = u32_np(k, np.arange(n, dtype=np.uint64))
    return (lo + ((u * np.uint64(hi - lo)) >> np.uint64(32)).astype(np.int64)).astype(np.int64)


def embed_np(E_kn, M_gn):
    """Q16 embedding rows (V, D) from the int8 table in (K=D, N=V) layout: rint(E * M / 2^12)."""
    D, V = E_kn.shape
    Mk = np.repeat(M_gn, 128, axis=0)                       # (D, V)
    a = E_kn.astype(np.int64) * Mk
    q = a >> 12
    rem = a & 4095
    q = q + ((rem > 2048) | ((rem == 2048) & ((q & 1) == 1)))
    return q.T.astype(np.int64)


# ----------------------------------------------------------------------------- tensor inventory
def linear_specs(cfg, li):
    """(name, N, K, bias) of the linears of layer li (output features N, input features K)."""
    D, H, KV, hd = cfg.D, cfg.H, cfg.KV, cfg.hd
    s = [(f"L{li}.q", H * hd, D, True), (f"L{li}.k", KV * hd, D, True), (f"L{li}.v", KV * hd, D, True),
         (f"L{li}.o", D, H * hd, False)]
    if cfg.moe:
        s.append((f"L{li}.router", cfg.NE, D, False))
        for e in range(cfg.NE):
            s += [(f"L{li}.e{e}.gate", cfg.MI, D, False), (f"L{li}.e{e}.up", cfg.MI, D, False),
                  (f"L{li}.e{e}.down", D, cfg.MI, False)]
        s += [(f"L{li}.sg", cfg.SI, D, False), (f"L{li}.su", cfg.SI, D, False), (f"L{li}.sd", D, cfg.SI, False),
              (f"L{li}.sgate", 1, D, False)]
    else:
        s += [(f"L{li}.gate", cfg.I, D, False), (f"L{li}.up", cfg.I, D, False), (f"L{li}.down", D, cfg.I, False)]
    return s


def arrays(cfg, seed):
    """Host integer arrays (DeviceWeights.from_arrays layout) of the dense synthetic model (cfg, seed): the same
    integers DeviceWeights.synthetic generates on the device."""
    if cfg.moe:
        raise ValueError("dense models only")
    out = {}
    for li in range(cfg.NL):
        out[f"{li}.g1"] = vector_np(key(seed, f"L{li}.g1"), cfg.D, *GAIN)
        out[f"{li}.g2"] = vector_np(key(seed, f"L{li}.g2"), cfg.D, *GAIN)
        for name, N, K, bias in linear_specs(cfg, li):
            short = name.split(".", 1)[1]
            out[f"{li}.{short}.w"] = weights_np(key(seed, name + ".w"), N, K)
            out[f"{li}.{short}.M"] = scales_np(key(seed, name + ".m"), N, K)
            if bias:
                out[f"{li}.{short}.b"] = vector_np(key(seed, name + ".b"), N, *BIAS)
    ew, eM = weights_np(key(seed, "emb.w"), cfg.V, cfg.D), scales_np(key(seed, "emb.m"), cfg.V, cfg.D)
    out["emb"] = embed_np(ew, eM)
    out["gf"] = vector_np(key(seed, "gf"), cfg.D, *GAIN)
    if cfg.tie:
        out["head.w"], out["head.M"] = ew, eM
    else:
        out["head.w"] = weights_np(key(seed, "head.w"), cfg.V, cfg.D)
        out["head.M"] = scales_np(key(seed, "head.m"), cfg.V, cfg.D)
    return out


def head_name(cfg):
    return "emb" if cfg.tie else "head"


def param_bytes(cfg):
    """int8 weight bytes + int16 scale bytes of the linears (layers + head)."""
    tot = 0
    for li in range(cfg.NL):
        for _, N, K, _b in linear_specs(cfg, li):
            tot += N * K + N * (K // 128) * 2
    return tot + cfg.V * cfg.D + cfg.V * (cfg.D // 128) * 2


def digest(arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]
