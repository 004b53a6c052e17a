"""The bundle format (FORMAT.md v1; src/bundle.rs:314-376, src/convert.rs:
124-366): the writer's manifest follows the format, the library's reader
(host only, no device) gives back every array byte for byte, and refuses
what the reference refuses."""
import json
import os

import numpy as np
import pytest

import fieldrun_amd as fa
from fieldrun_amd import convert
from fieldrun_amd.bundle import BundleWriter, manifest


def write_sample(stem):
    rng = np.random.default_rng(3)
    w = BundleWriter(stem)
    wte = rng.standard_normal((50, 16)).astype(np.float32)
    w.put_embed("wte", wte, "int8")
    w.put_small("wpe", rng.standard_normal((8, 16)), None, "f32")
    w.put_small("ln.weight", rng.standard_normal(16), None, "f16")
    lin = rng.standard_normal((24, 16)).astype(np.float32)       # (out, in)
    w.put_lin("h0.attn.c_attn.weight", lin, "int8")
    w.put_lin("h0.mlp.c_fc.weight", rng.standard_normal((12, 37)), "int4")   # odd in: packed tail
    w.put_lin("h0.mlp.c_proj.weight", rng.standard_normal((16, 12)), "f16")
    w.put_i8("l0.experts.0.gate", rng.standard_normal((16, 8)), False)       # (in, out) source
    w.finish(manifest("gpt2", [1, 2, 16, 8, 50], eos=[49]))
    return wte, lin


def test_writer_manifest_follows_the_format(tmp_path):
    stem = str(tmp_path / "m")
    write_sample(stem)
    m = json.load(open(stem + ".fieldrun.json"))
    assert m["format"] == "fieldrun-bundle" and m["version"] == 1 and m["arch"] == "gpt2"
    assert m["config"] == [1, 2, 16, 8, 50] and m["eos"] == [49]
    off = 0
    size = {"f32": 4, "f16": 2, "i8": 1, "rowi8": 1}
    for a in m["arrays"]:
        assert a["offset"] == off                        # blob order, contiguous
        if a["dtype"] == "i4":
            assert a["bytes"] == a["shape"][0] * ((a["shape"][1] + 1) // 2) and a["group"] == 32
        else:
            assert a["bytes"] == int(np.prod(a["shape"])) * size[a["dtype"]] and "group" not in a
        off += a["bytes"]
    assert off == os.path.getsize(stem + ".fieldrun.bin")
    names = [a["name"] for a in m["arrays"]]
    # every quantised array is followed by its f16 scale sibling (convert.rs)
    for a in m["arrays"]:
        if a["dtype"] in ("i8", "i4", "rowi8"):
            s = m["arrays"][names.index(a["name"]) + 1]
            assert s["name"] == a["name"] + "__scale" and s["dtype"] == "f16"
    dt = {a["name"]: (a["dtype"], a["shape"]) for a in m["arrays"]}
    assert dt["h0.attn.c_attn.weight"] == ("i8", [16, 24])       # stored (in, out)
    assert dt["h0.mlp.c_fc.weight"] == ("i4", [12, 37])          # stored (out, in)
    assert dt["h0.mlp.c_proj.weight"] == ("f16", [12, 16])       # transposed to (in, out)
    assert dt["wte"] == ("rowi8", [50, 16])


def test_reader_round_trip(tmp_path):
    stem = str(tmp_path / "m")
    wte, lin = write_sample(stem)
    b = fa.Bundle(stem)
    assert b.arch == "gpt2" and b.config == [1, 2, 16, 8, 50] and b.config_f == []
    m = json.load(open(stem + ".fieldrun.json"))
    blob = open(stem + ".fieldrun.bin", "rb").read()
    for a in m["arrays"]:
        dt, shape, group, nb = b.info(a["name"])
        assert (dt, list(shape), nb) == (a["dtype"], a["shape"], a["bytes"])
        assert group == a.get("group", 0)
        raw = b.arr(a["name"]).tobytes()
        assert raw == blob[a["offset"]:a["offset"] + a["bytes"]]
    q, s16 = convert.put_embed_i8(wte)
    assert np.array_equal(b.arr("wte"), q)
    assert np.array_equal(b.arr("wte__scale"), s16)
    w8, s8 = convert.put_i8(lin, True)
    assert np.array_equal(b.arr("h0.attn.c_attn.weight"), w8)
    assert b.dims("h0.attn.c_attn.weight") == (16, 24)
    with pytest.raises(fa.FrqError) as e:
        b.info("nope")
    assert e.value.code == fa.FRQ_ERR_MISSING and "missing array nope" in str(e.value)
    with pytest.raises(fa.FrqError):
        b.weight("wte")   # no device context
    b.close()


def write_manifest(stem, m, blob=b"\0" * 64):
    with open(stem + ".fieldrun.json", "w") as f:
        f.write(m if isinstance(m, str) else json.dumps(m))
    with open(stem + ".fieldrun.bin", "wb") as f:
        f.write(blob)


def base():
    return {"format": "fieldrun-bundle", "version": 1, "arch": "rope", "config": [1, 2, 3],
            "arrays": [{"name": "a", "dtype": "f32", "shape": [4, 4], "offset": 0, "bytes": 64}]}


@pytest.mark.parametrize("edit,code", [
    (lambda m: m.update(format="fieldrun"), fa.FRQ_ERR_FORMAT),
    (lambda m: m.update(version=2), fa.FRQ_ERR_FORMAT),
    (lambda m: m["arrays"][0].update(offset=8), fa.FRQ_ERR_FORMAT),        # past the blob
    (lambda m: m["arrays"][0].update(bytes=1 << 62), fa.FRQ_ERR_FORMAT),
    (lambda m: m["arrays"][0].update(shape=[-1]), fa.FRQ_ERR_FORMAT),
    (lambda m: m.pop("arrays"), fa.FRQ_ERR_FORMAT),
    (lambda m: m.update(config=[1.5]), fa.FRQ_ERR_FORMAT),
])
def test_reader_refuses_what_the_reference_refuses(tmp_path, edit, code):
    stem = str(tmp_path / "m")
    m = base()
    edit(m)
    write_manifest(stem, m)
    with pytest.raises(fa.FrqError) as e:
        fa.Bundle(stem)
    assert e.value.code == code


def test_reader_message_and_io_errors(tmp_path):
    stem = str(tmp_path / "m")
    m = base()
    m["version"] = 7
    write_manifest(stem, m)
    with pytest.raises(fa.FrqError) as e:
        fa.Bundle(stem)
    assert "unsupported bundle: fieldrun-bundle v7" in str(e.value)
    for bad in ['{"format": "fieldrun-bundle", "version": 1,', '[1, 2', '{"a" 1}', '{"a": tru}', '{} x']:
        write_manifest(stem, bad)
        with pytest.raises(fa.FrqError) as e:
            fa.Bundle(stem)
        assert e.value.code == fa.FRQ_ERR_FORMAT
    with pytest.raises(fa.FrqError) as e:
        fa.Bundle(str(tmp_path / "absent"))
    assert e.value.code == fa.FRQ_ERR_ARG


def test_reader_json_details(tmp_path):
    # default dtype f32, group null, escapes and unicode in names, a nested
    # store, floats with exponents, and whitespace everywhere
    stem = str(tmp_path / "m")
    text = ('\n { "store" : {"quad": [[1, 2, {"x": null}], -3.5e-2], "s": "\\u00e9\\"\\\\"},\n'
            '  "format":"fieldrun-bundle","version":1,"arch":"gemma","config":[ 26 , 8 ,-1 ],\n'
            '  "config_f":[1e4, 1.0E-6, 50, -0.25],\n'
            '  "arrays":[{"name":"emb\\u00e9d\\t","shape":[2,8],"offset":0,"bytes":64,"group":null}] }\n')
    write_manifest(stem, text)
    b = fa.Bundle(stem)
    assert b.arch == "gemma" and b.config == [26, 8, -1]
    assert b.config_f == [1e4, 1e-6, 50.0, -0.25]
    dt, shape, group, nb = b.info("embéd\t")
    assert (dt, shape, group, nb) == ("f32", (2, 8), 0, 64)
    b.close()


def test_config_bundles_follow_the_converters(tmp_path):
    """The synthetic config bundles carry the names, dtypes and stored
    shapes convert_gpt2 (src/convert.rs:505-545) and convert_qwen3moe
    (872-938, one MoE layer) write for an int8 build."""
    from fieldrun_amd import synth
    stem = str(tmp_path / "g")
    synth.write_gpt2_bundle(stem, 1, n_layer=2, n_head=2, d=32, n_pos=8, vocab=40)
    m = json.load(open(stem + ".fieldrun.json"))
    assert (m["arch"], m["config"]) == ("gpt2", [2, 2, 32, 8, 40])
    dt = {a["name"]: (a["dtype"], a["shape"]) for a in m["arrays"]}
    want = {"wte": ("f16", [40, 32]), "wpe": ("f16", [8, 32]),
            "ln_f.weight": ("f16", [32]), "ln_f.bias": ("f16", [32])}
    for l in range(2):
        for ln in ("ln_1", "ln_2"):
            want[f"h{l}.{ln}.weight"] = want[f"h{l}.{ln}.bias"] = ("f16", [32])
        for name, (i, o) in (("attn.c_attn", (32, 96)), ("attn.c_proj", (32, 32)),
                             ("mlp.c_fc", (32, 128)), ("mlp.c_proj", (128, 32))):
            want[f"h{l}.{name}.weight"] = ("i8", [i, o])
            want[f"h{l}.{name}.weight__scale"] = ("f16", [o])
            want[f"h{l}.{name}.bias"] = ("f16", [o])
    assert dt == want
    b = fa.Bundle(stem)
    assert np.all(b.arr("h1.ln_2.weight") == 1) and np.all(b.arr("h0.attn.c_proj.bias") == 0)
    b.close()

    stem = str(tmp_path / "q")
    synth.write_qwen3moe_layer_bundle(stem, 1, n_exp=3, d=64, mi=16, topk=2)
    m = json.load(open(stem + ".fieldrun.json"))
    assert m["arch"] == "qwen3moe" and m["config_f"] == [1e6, 1e-6]
    # [nl, nh, nkv, hd, d, ffn, vocab, tie, n_exp, topk, moe_inter, norm_topk, moe flag l0, window]
    assert m["config"] == [1, 32, 4, 128, 64, 6144, 151936, 0, 3, 2, 16, 1, 1, 0]
    dt = {a["name"]: (a["dtype"], a["shape"]) for a in m["arrays"]}
    want = {"l0.gate": ("i8", [64, 3]), "l0.gate__scale": ("f16", [3])}
    for e in range(3):
        for fr, (i, o) in (("gate", (64, 16)), ("up", (64, 16)), ("down", (16, 64))):
            want[f"l0.experts.{e}.{fr}"] = ("i8", [i, o])
            want[f"l0.experts.{e}.{fr}__scale"] = ("f16", [o])
    assert dt == want
