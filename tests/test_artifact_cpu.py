"""The on-disk exact artifact (SPEC.md:7-12) on the host: round trip, manifest hashes, tamper detection, and the
synthetic arrays it is written from (the same integers as the oracle-side generator)."""
import hashlib
import json
import os

import numpy as np
import pytest

import helpers
from exact_amd import artifact, synth, tables
from exact_amd.ops import ExactError


def _write(tmp_path, name="tiny", mode="group"):
    cfg = synth.CONFIGS[name]
    arr = synth.arrays(cfg, 9)
    tab = tables.host_tables(64, cfg.hd, cfg.theta)
    man = artifact.write(str(tmp_path), cfg, arr, tab, mode=mode)
    return cfg, arr, tab, man


def test_synthetic_arrays_are_the_generator_integers():
    cfg = synth.CONFIGS["tiny"]
    arr = synth.arrays(cfg, 9)
    ow = helpers.oracle_weights(cfg, 9)
    for i, L in enumerate(ow["layers"]):
        for k in ("q", "k", "v", "o", "gate", "up", "down"):
            assert np.array_equal(arr[f"{i}.{k}.w"], L[k].w) and np.array_equal(arr[f"{i}.{k}.M"], L[k].M)
            assert (L[k].b is None) == (f"{i}.{k}.b" not in arr)
        assert np.array_equal(arr[f"{i}.g1"], L["g1"]) and np.array_equal(arr[f"{i}.g2"], L["g2"])
    assert np.array_equal(arr["emb"], ow["emb"]) and np.array_equal(arr["gf"], ow["gf"])
    assert np.array_equal(arr["head.w"], ow["head"].w) and np.array_equal(arr["head.M"], ow["head"].M)


@pytest.mark.parametrize("name,mode", [("tiny", "group"), ("tiny-tied", "channel")])
def test_round_trip(tmp_path, name, mode):
    cfg, arr, tab, man = _write(tmp_path, name, mode)
    cfg2, mode2, arr2, tab2 = artifact.load(str(tmp_path))
    assert cfg2 == cfg and mode2 == mode
    assert sorted(arr2) == sorted(arr)
    for k in arr:
        assert np.array_equal(arr2[k], arr[k]), k
    for k in artifact.TABLES:
        assert np.array_equal(tab2[k], tab[k]), k
    assert np.array_equal(tab2["exp"], tables.exp_t()) and np.array_equal(tab2["silu"], tables.silu_t())
    assert arr2["0.q.w"].dtype == np.int8 and arr2["emb"].dtype == np.int32 and arr2["0.q.M"].dtype == np.int64


def test_manifest_hashes_and_layout(tmp_path):
    cfg, arr, tab, man = _write(tmp_path)
    on_disk = json.load(open(os.path.join(str(tmp_path), "manifest.json")))
    assert on_disk == json.loads(json.dumps(man))
    assert on_disk["spec"] == "0.4" and on_disk["format"] == "Q16"
    for f in artifact.FILES:
        data = open(os.path.join(str(tmp_path), f), "rb").read()
        assert on_disk["files"][f]["sha256"] == hashlib.sha256(data).hexdigest()
        assert on_disk["files"][f]["bytes"] == len(data)
    # weights.int8 holds exactly the int8 matrices, in the manifest's order
    wbytes = sum(a.size for k, a in arr.items() if k.endswith(".w"))
    assert on_disk["files"]["weights.int8"]["bytes"] == wbytes
    e = next(x for x in on_disk["arrays"] if x["name"] == "0.k.w")
    raw = open(os.path.join(str(tmp_path), "weights.int8"), "rb").read()
    got = np.frombuffer(raw[e["offset"]:e["offset"] + arr["0.k.w"].size], np.int8).reshape(e["shape"])
    assert np.array_equal(got, arr["0.k.w"])


def test_tampered_files_are_rejected(tmp_path):
    _write(tmp_path)
    p = os.path.join(str(tmp_path), "weights.int8")
    b = bytearray(open(p, "rb").read())
    b[12345] ^= 1
    open(p, "wb").write(bytes(b))
    with pytest.raises(ExactError, match="SHA-256"):
        artifact.load(str(tmp_path))
    artifact.load(str(tmp_path), verify=False)          # the caller may skip the check explicitly
    os.truncate(os.path.join(str(tmp_path), "tables.int"), 8)
    with pytest.raises(ExactError, match="size"):
        artifact.load(str(tmp_path), verify=False)


def test_writer_rejects_non_integer_and_out_of_range(tmp_path):
    cfg = synth.CONFIGS["tiny"]
    arr = synth.arrays(cfg, 9)
    tab = tables.host_tables(64, cfg.hd, cfg.theta)
    bad = dict(arr)
    bad["gf"] = arr["gf"].astype(np.float64)
    with pytest.raises(ExactError, match="integer"):
        artifact.write(str(tmp_path / "a"), cfg, bad, tab)
    bad = dict(arr)
    bad["emb"] = arr["emb"] * (1 << 30)
    with pytest.raises(ExactError, match="fit"):
        artifact.write(str(tmp_path / "b"), cfg, bad, tab)


def test_manifest_that_points_elsewhere_is_rejected(tmp_path):
    """The loader maps only the hash-checked files, with known dtypes and extents inside each file."""
    import json
    _write(tmp_path)
    mp = os.path.join(str(tmp_path), "manifest.json")
    good = json.load(open(mp))

    def load_with(edit):
        man = json.loads(json.dumps(good))
        edit(man)
        json.dump(man, open(mp, "w"))
        return artifact.load(str(tmp_path), verify=False)

    with pytest.raises(ExactError, match="lists files"):
        load_with(lambda m: m["files"].pop("tables.int"))
    with pytest.raises(ExactError, match="outside the artifact"):
        load_with(lambda m: m["arrays"][0].update(file="../manifest.json"))
    with pytest.raises(ExactError, match="dtype"):
        load_with(lambda m: m["arrays"][0].update(dtype="<f8"))
    with pytest.raises(ExactError, match="past the end"):
        load_with(lambda m: m["arrays"][0].update(offset=good["files"][good["arrays"][0]["file"]]["bytes"]))
    json.dump(good, open(mp, "w"))
    artifact.load(str(tmp_path))
