"""The on-disk exact artifact (SPEC.md:7-12): weights.int8 + scales.int + tables.int + manifest.json, all
values integers, the tables shipped rather than recomputed, and the SHA-256 of every file in the manifest.

The reference specifies the artifact but ships no writer or loader for it; this is one, in this layout:
  weights.int8   every linear's int8 weight matrix W (K, N) (the reference's QLin / GQLin `w`,
                 exact_llm.py:82-96), row-major, one after another;
  scales.int     every other integer array, little-endian, each with its own width: group scales M (K/128, N)
                 or channel scales M (N,) as int64, biases and norm gains (Q16) as int64, the embedding rows
                 (V, D, Q16) as int32;
  tables.int     int64 little-endian: exp (10242, Q24), silu (8194, Q16), sig (8194, Q16), RoPE cos and sin
                 (T, hd, Q16) for T positions;
  manifest.json  spec version, fixed-point format, architecture, linear mode, table ids, and for every array
                 its file, byte offset, dtype and shape, and for every file its size and SHA-256.
Array names follow DeviceWeights.from_arrays: emb, gf, head.w / head.M (/ head.b), and per layer i
f"{i}.g1", f"{i}.g2", f"{i}.{q|k|v|o|gate|up|down}.w" / ".M" / ".b".
"""
import hashlib
import json
import os

import numpy as np

from ._lib import ExactError
from .synth import ModelConfig

SPEC_VERSION = "0.4"
FILES = ("weights.int8", "scales.int", "tables.int")
TABLES = ("exp", "silu", "sig", "cos", "sin")
_DT = {"i1": np.int8, "<i2": np.int16, "<i4": np.int32, "<i8": np.int64}


def _sha256_file(path, chunk=1 << 24):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(chunk)
            if not b:
                return h.hexdigest()
            h.update(b)


def _names(cfg):
    names = ["emb", "gf"]
    for i in range(cfg.NL):
        names += [f"{i}.g1", f"{i}.g2"]
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            names += [f"{i}.{k}.w", f"{i}.{k}.M", f"{i}.{k}.b"]
    return names + ["head.w", "head.M", "head.b"]


def write(path, cfg, arrays, tables, mode="group"):
    """Write an artifact directory from integer arrays (DeviceWeights.from_arrays layout) and host tables
    (tables.host_tables). Returns the manifest."""
    if cfg.moe:
        raise ExactError("the artifact layout covers dense models")
    if mode not in ("group", "channel"):
        raise ExactError(f"linear mode {mode!r}")
    os.makedirs(path, exist_ok=True)
    index, offs = [], {f: 0 for f in FILES}
    handles = {f: open(os.path.join(path, f), "wb") for f in FILES}
    try:
        def put(name, a, fname, dt):
            a = np.asarray(a)
            if not np.issubdtype(a.dtype, np.integer):
                raise ExactError(f"{name}: integer array expected, got {a.dtype}")
            b = np.ascontiguousarray(a.astype(_DT[dt], copy=False))
            if not np.array_equal(b, a):
                raise ExactError(f"{name}: values do not fit {dt}")
            handles[fname].write(memoryview(np.ascontiguousarray(b, dtype=np.dtype(dt))).cast("B"))
            index.append(dict(name=name, file=fname, offset=offs[fname], dtype=dt, shape=list(a.shape)))
            offs[fname] += b.nbytes

        for name in _names(cfg):
            if name not in arrays:
                if name.endswith(".b"):
                    continue
                raise ExactError(f"missing array {name}")
            if name.endswith(".w"):
                put(name, arrays[name], "weights.int8", "i1")
            else:
                put(name, arrays[name], "scales.int", "<i4" if name == "emb" else "<i8")
        for t in TABLES:
            put(t, tables[t], "tables.int", "<i8")
    finally:
        for h in handles.values():
            h.close()
    manifest = dict(
        spec=SPEC_VERSION, format="Q16",
        architecture=dict(name=cfg.name, layers=cfg.NL, hidden=cfg.D, heads=cfg.H, kv_heads=cfg.KV, head_dim=cfg.hd,
                          intermediate=cfg.I, vocab=cfg.V, rope_theta=cfg.theta, tied_head=cfg.tie),
        linear_mode=mode,
        head_mode="group" if np.ndim(arrays["head.M"]) == 2 else "channel",
        tables=dict(exp="Q24 exp(-i/256), i < 10242", silu="Q16 SiLU on [-16, 16) at 1/256 steps",
                    sig="Q16 sigmoid on [-16, 16) at 1/256 steps", cos="Q16 RoPE cos (T, hd)", sin="Q16 RoPE sin (T, hd)"),
        arrays=index,
        files={f: dict(bytes=offs[f], sha256=_sha256_file(os.path.join(path, f))) for f in FILES})
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    return manifest


def load(path, verify=True):
    """(cfg, mode, arrays, tables) of an artifact directory; arrays are read-only memory maps. verify checks
    every file's size and SHA-256 against the manifest first and raises ExactError on any mismatch."""
    try:
        with open(os.path.join(path, "manifest.json")) as f:
            man = json.load(f)
    except (OSError, ValueError) as e:
        raise ExactError(f"artifact manifest unreadable: {e}") from None
    if man.get("spec") != SPEC_VERSION or man.get("format") != "Q16":
        raise ExactError(f"artifact spec {man.get('spec')!r} / format {man.get('format')!r} not supported")
    if set(man.get("files", {})) != set(FILES):
        raise ExactError(f"artifact manifest lists files {sorted(man.get('files', {}))}, expected {sorted(FILES)}")
    for fname, meta in man["files"].items():
        fp = os.path.join(path, fname)
        if not os.path.exists(fp) or os.path.getsize(fp) != meta["bytes"]:
            raise ExactError(f"{fname}: missing or wrong size")
        if verify and _sha256_file(fp) != meta["sha256"]:
            raise ExactError(f"{fname}: SHA-256 differs from the manifest")
    a = man["architecture"]
    cfg = ModelConfig(a["name"], D=a["hidden"], H=a["heads"], KV=a["kv_heads"], hd=a["head_dim"], I=a["intermediate"],
                      V=a["vocab"], NL=a["layers"], theta=a["rope_theta"], tie=a["tied_head"])
    maps, arrays, tables = {}, {}, {}
    for e in man["arrays"]:
        if e["file"] not in FILES:      # only the size- and hash-checked files above, never another path
            raise ExactError(f"array {e.get('name')!r} names file {e['file']!r} outside the artifact")
        if e["dtype"] not in _DT:
            raise ExactError(f"array {e.get('name')!r} has dtype {e['dtype']!r}")
        if e["file"] not in maps:
            maps[e["file"]] = np.memmap(os.path.join(path, e["file"]), dtype=np.uint8, mode="r")
        dt = np.dtype(e["dtype"])
        n = int(np.prod(e["shape"])) if e["shape"] else 1
        off = int(e["offset"])
        if off < 0 or n < 0 or off + n * dt.itemsize > maps[e["file"]].size:
            raise ExactError(f"array {e.get('name')!r} runs past the end of {e['file']}")
        raw = maps[e["file"]][off:off + n * dt.itemsize]
        arr = raw.view(dt).reshape(e["shape"])
        (tables if e["file"] == "tables.int" else arrays)[e["name"]] = arr
    return cfg, man["linear_mode"], arrays, tables
