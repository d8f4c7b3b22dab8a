"""The geode-pack reader (gv_pack_*, host calls: no GPU) against the manifests and files of tests/pack_writer.py: the
tensor table as Python's own json reads it, the expert table, the refusals of Pack::open (engine/src/pack.cpp:39-308)
one planted damage each, the pack print (FNV-1a of geode.json from the reference's start), and the tile8 layout
against the reference's own to_tile8 (golden fixture) in both directions."""
import json
import os

import numpy as np
import pytest

import pyoracle as po
import state_format as sf
from pack_writer import to_tile8, write_pack

CFG = dict(hidden=128, vocab=256, n_layers=2, n_experts=8, top_k=2, moe_ff=64, shared_ff=64, n_heads=4, n_kv_heads=2,
           head_dim=32, rope_dim=16, rope_theta=1e4, eps=1e-6, max_ctx=96)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    return geode_amd


@pytest.fixture(scope="module")
def om():
    return po.Model(CFG, seed=5, ctx=0)


@pytest.mark.parametrize("name", ["tile8_a", "tile8_b"])
def test_tile8_against_the_reference(gv, name):
    g = np.load(GOLDEN)
    rows, tiled = g[name + "_rows"], g[name + "_tiled"]
    r, c = rows.shape[0], rows.shape[1] // 9 * 16
    assert np.array_equal(to_tile8(r, c, rows), tiled)                    # the test's writer = the reference's
    assert np.array_equal(gv.q4_untile8(r, c, tiled).reshape(rows.shape), rows)   # the library's inverse
    if name == "tile8_b":
        assert np.array_equal(g["tile8_b_row37"], rows[37])


def test_tile8_round_trip_random_bytes(gv):
    rng = np.random.default_rng(3)
    rows, cols = 64, 256
    m = rng.integers(0, 256, (rows, cols // 16 * 9), dtype=np.uint8)
    assert np.array_equal(gv.q4_untile8(rows, cols, to_tile8(rows, cols, m)).reshape(m.shape), m)


@pytest.mark.parametrize("tile8", [False, True])
def test_open_reads_the_tables(gv, om, tmp_path, tile8):
    m = write_pack(om, str(tmp_path), tile8=tile8)
    p = gv.Pack(str(tmp_path))
    assert p.tile8 == tile8
    text = open(tmp_path / "geode.json", "rb").read()
    assert p.print == sf.fnv1a(text)
    files = [f["name"] for f in m["files"]]
    for name, t in m["tensors"].items():
        got = p.tensor(name)
        shape = t["shape"]
        rows, cols = (1, shape[0]) if len(shape) == 1 else (shape[0], int(np.prod(shape[1:])))
        assert (got["type"], got["rows"], got["cols"], got["file"], got["offset"]) == \
               (t["type"], rows, cols, files.index(t["file"]), t["offset"]), name
        assert got["global"] == np.float32(t.get("global", 1.0))
    for l, layer in enumerate(m["experts"]["layers"]):
        for e in (0, 3, CFG["n_experts"] - 1):
            assert p.expert(l, e) == (files.index("experts.bin"), layer["offset"] + e * layer["stride"], "q4")
    cfg = p.model_config(max_ctx=96, max_rows=17)
    for k in ("hidden", "vocab", "n_layers", "n_experts", "top_k", "moe_ff", "shared_ff", "n_heads", "n_kv_heads",
              "head_dim", "rope_dim"):
        assert cfg[k] == CFG[k], k
    assert cfg["rope_theta"] == np.float32(CFG["rope_theta"]) and cfg["eps"] == np.float32(CFG["eps"])
    assert cfg["mtp"] == 0


def test_mtp_pack_tables(gv, tmp_path):
    """a pack with an MTP layer: the manifest's "mtp" experts are expert layer n_layers (pack.cpp:303-305, Pack::expert
    past the main layers), its tensors are in the table, and the config asks for the MTP layer"""
    om = po.Model(dict(CFG, mtp=1), seed=4)
    m = write_pack(om, str(tmp_path))
    p = gv.Pack(str(tmp_path))
    files = [f["name"] for f in m["files"]]
    for e in (0, CFG["n_experts"] - 1):
        assert p.expert(CFG["n_layers"], e) == (files.index("experts.bin"),
                                                m["mtp"]["experts"]["offset"] + e * m["mtp"]["experts"]["stride"], "q4")
    assert p.tensor("mtp.fc.weight")["cols"] == 2 * CFG["hidden"]
    assert p.model_config(96)["mtp"] == 1


def _damage(what):
    def mutate(m):
        if what == "format":
            m["format"] = "other"
        elif what == "version":
            m["version"] = 2
        elif what == "arch":
            m["arch"] = "llama"
        elif what == "size":
            m["files"][0]["size"] += 1
        elif what == "layers":
            m["config"]["layer_types"] = m["config"]["layer_types"][:1]
        elif what == "geometry":
            m["config"]["hidden_size"] = 130
        elif what == "type":
            m["tensors"]["norm.weight"]["type"] = "f64"
        elif what == "past_end":
            m["tensors"]["lm_head.weight"]["offset"] = m["files"][0]["size"] - 8
        elif what == "negative":
            m["tensors"]["lm_head.weight"]["offset"] = -1
        elif what == "cols":
            m["tensors"]["lm_head.weight"]["shape"] = [256, 120]
        elif what == "unlisted":
            m["tensors"]["norm.weight"]["file"] = "other.bin"
        elif what == "no_dense":
            for t in m["tensors"].values():
                t["file"] = "experts.bin"
        elif what == "embed":
            del m["tensors"]["embed_tokens.weight"]
        elif what == "experts":
            m["experts"]["layers"] = m["experts"]["layers"][:1]
        elif what == "scales":
            del m["tensors"]["layers.1.mlp.experts.scales"]
        elif what == "expert_count":
            e = m["experts"]["layers"][0]
            m["experts"]["layers"][0] = {"file": e["file"], "offsets": [e["offset"]] * 3, "formats": ["q4"] * 3}
    return mutate


@pytest.mark.parametrize("what,message", [
    ("format", "format 'other' version 1; this reader takes geode-pack version 1"),
    ("version", "format 'geode-pack' version 2;"), ("arch", "architecture 'llama' is not one this library loads"),
    ("size", "bytes; geode.json lists"), ("layers", "layer_types lists 1 layers"),
    ("geometry", "model geometry: hidden_size 130"), ("type", "type 'f64' is not a known tensor type"),
    ("past_end", "its bytes run past the end of dense.bin"), ("negative", "outside what a pack can hold"),
    ("cols", "needs a multiple of 16 columns"), ("unlisted", "file 'other.bin' is not one of geode.json's files"),
    ("no_dense", "no tensor in dense.bin"), ("embed", "embed_tokens.weight must be"),
    ("experts", "expert table has 1 layers; the model has 2"), ("scales", "layer 1: the scales tensor"),
    ("expert_count", "3 experts listed, config.num_experts is 8")])
def test_open_refuses(gv, om, tmp_path, what, message):
    write_pack(om, str(tmp_path), mutate=_damage(what))
    with pytest.raises(gv.GeodeError, match=message):
        gv.Pack(str(tmp_path))


def test_json_reader_against_pythons(gv, om, tmp_path):
    """a manifest with escapes, unicode (\\u and raw UTF-8, a surrogate pair), exponents and odd spacing: the names and
    numbers the library reads are those Python's json reads"""
    m = write_pack(om, str(tmp_path))
    odd = {"läyer \"x\"\\\t€\U0001F600": dict(m["tensors"]["norm.weight"]),
           "plain": dict(m["tensors"]["norm.weight"], global_=1)}
    odd["plain"]["global"] = 2.5e-3
    m["tensors"].update(odd)
    text = json.dumps(m, ensure_ascii=True, indent=None, separators=(" ,", " :  "))
    assert '"global" :  0.0025' in text
    text = text.replace('"global" :  0.0025', '"global":2.5E-3')
    with open(tmp_path / "geode.json", "w") as f:
        f.write(text)
    p = gv.Pack(str(tmp_path))
    got = p.tensor("läyer \"x\"\\\t€\U0001F600")
    assert got["offset"] == m["tensors"]["norm.weight"]["offset"]
    assert p.tensor("plain")["global"] == np.float32(2.5e-3)


GDN_CFG = dict(CFG, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
               gdn_layers=[1, 0, 1])


def test_gated_deltanet_pack(gv, tmp_path):
    """a pack of Gated DeltaNet layers (layer_types "linear_attention", the linear_* shape, pack.cpp:96-100): the
    GPU config takes its shape and layers, its linear_attn tensors are where the manifest says"""
    om = po.Model(GDN_CFG, seed=6, ctx=0)
    m = write_pack(om, str(tmp_path))
    p = gv.Pack(str(tmp_path))
    cfg = p.model_config(96)
    for k in ("gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim", "conv_kernel", "gdn_layers"):
        assert cfg[k] == GDN_CFG[k], k
    conv = p.tensor("layers.0.linear_attn.conv1d.weight")
    assert (conv["type"], conv["rows"], conv["cols"]) == ("f32", 256, 4)   # [conv_dim, 1, K]: rows, the rest
    t = m["tensors"]["layers.2.linear_attn.in_proj_qkv.weight"]
    got = p.tensor("layers.2.linear_attn.in_proj_qkv.weight")
    assert (got["rows"], got["cols"], got["offset"]) == (256, 128, t["offset"])
    assert got["global"] == np.float32(om.tensor(po.GDN_QKV, 2)[1][0])
    with pytest.raises(gv.GeodeError, match="no layers.0.self_attn"):
        p.tensor("layers.0.self_attn.q_proj.weight")


@pytest.mark.parametrize("text,valid", [
    ('{"a": [1, 2,]}', False), ('{"a": 01}', False), ('{"a": 1.}', False), ('{"a": -}', False),
    ('{"a": "\\ud800"}', False), ('{"a": "\\udc00\\ud800"}', False), ('{"a": "x\ty"}', False),
    ('{"a": "\\x"}', False), ('{"a" 1}', False), ('{"a": 1} {}', False), ('{"a": [1 2]}', False),
    ('{"a": tru}', False), ('{"a": "open}', False), ('[', False), ('', False),
    ('{"a": [], "b": {}, "c": [[], {}], "d": -0, "e": 1E+2, "f": 0.5e-3, "g": "\\ud83d\\ude00", "h": null}', True),
    ('  {"format": "geode-pack", "version": 1}\n', True)])
def test_json_reader_follows_rfc_8259(gv, tmp_path, text, valid):
    """the manifest reader accepts RFC 8259's grammar and nothing else: a document it refuses is reported as invalid
    JSON; one it accepts goes on to the manifest's own checks (which these minimal documents then fail)"""
    (tmp_path / "geode.json").write_text(text, encoding="utf-8")
    with pytest.raises(gv.GeodeError) as e:
        gv.Pack(str(tmp_path))
    assert ("is not valid JSON" in str(e.value)) != valid, str(e.value)
