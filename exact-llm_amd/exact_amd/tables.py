"""Integer tables shipped with an exact model (SPEC.md:11: tables ship as integers, never recomputed
per device). They are built once on the host from their closed forms with the same float64
expressions as the reference and then copied to the GPU, so every device reads the same integers.

  EXP_T   Q24 exp(-i/256), 10242 entries           exact_llm.py:107-108
  SILU_T  Q16 SiLU on [-16, 16) at 1/256 steps      exact_llm.py:116-117
  SIG_T   Q16 sigmoid on [-16, 16) at 1/256 steps   moe_exact_kaggle.py:419
  RoPE    Q16 cos/sin of pos * theta^(-2i/hd)       exact_llm.py:127-130,157-158
"""
import functools
import math

import numpy as np

ONE = 1 << 16


@functools.lru_cache(None)
def exp_t():
    return np.array([round(math.exp(-i / 256) * (1 << 24)) for i in range(256 * 40 + 2)], np.int64)


@functools.lru_cache(None)
def silu_t():
    vals = []
    for i in range(32 * 256 + 2):
        v = (i - 16 * 256) / 256
        vals.append(round(v / (1 + math.exp(-v)) * ONE))
    return np.array(vals, np.int64)


@functools.lru_cache(None)
def sig_t():
    return np.array([round(1.0 / (1.0 + math.exp(-((i - 16 * 256) / 256))) * ONE) for i in range(32 * 256 + 2)], np.int64)


def rope(T, hd, theta):
    """(cos, sin) int64 (T, hd) Q16."""
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.outer(np.arange(T, dtype=np.float64), inv)
    ang = np.concatenate([ang, ang], -1)
    return np.rint(np.cos(ang) * ONE).astype(np.int64), np.rint(np.sin(ang) * ONE).astype(np.int64)


def inv_sqrt_hd(hd):
    """Integer score scale C = round(2^16 / sqrt(hd)) (SPEC.md:22)."""
    return int(round((1 << 16) / math.sqrt(hd)))


def host_tables(T, hd, theta):
    """The tables of a model as host int64 arrays: exp, silu, sig, cos (T, hd), sin (T, hd)."""
    c, s = rope(T, hd, theta)
    return dict(exp=exp_t(), silu=silu_t(), sig=sig_t(), cos=c, sin=s)


class DeviceTables:
    """The tables as int32 / int64 device tensors."""

    def __init__(self, device, T, hd, theta):
        self._load(device, host_tables(T, hd, theta), T, hd)

    @classmethod
    def from_host(cls, device, tables, T, hd):
        """From given integer tables (an artifact's): RoPE rows for at least T positions."""
        self = cls.__new__(cls)
        self._load(device, tables, T, hd)
        return self

    def _load(self, device, tab, T, hd):
        import torch
        from ._lib import ExactError
        if len(tab["exp"]) != 256 * 40 + 2 or len(tab["silu"]) != 32 * 256 + 2 or len(tab["sig"]) != 32 * 256 + 2:
            raise ExactError("table sizes differ from the spec's (exp 10242, silu and sig 8194 entries)")
        if np.shape(tab["cos"])[0] < T or np.shape(tab["cos"])[1:] != (hd,) or np.shape(tab["sin"]) != np.shape(tab["cos"]):
            raise ExactError(f"RoPE tables need ({T}, {hd}) rows")
        if max(np.abs(np.asarray(tab[k], np.int64)).max() for k in ("exp", "silu", "sig")) >= 1 << 31:
            raise ExactError("exp/silu/sig tables must fit int32")
        self.exp = torch.tensor(np.asarray(tab["exp"], np.int64), dtype=torch.int32, device=device)
        self.silu = torch.tensor(np.asarray(tab["silu"], np.int64), dtype=torch.int32, device=device)
        self.sig = torch.tensor(np.asarray(tab["sig"], np.int64), dtype=torch.int32, device=device)
        self.cos = torch.tensor(np.asarray(tab["cos"], np.int64)[:T], dtype=torch.int64, device=device)
        self.sin = torch.tensor(np.asarray(tab["sin"], np.int64)[:T], dtype=torch.int64, device=device)
        self.T = T
        self.inv = inv_sqrt_hd(hd)
