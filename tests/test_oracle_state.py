"""The oracle's state file (oracle/oracle_state.cpp, a restatement of engine/src/state.cpp) pinned on the CPU:
FNV-1a against its published vectors, every byte of a save against the struct / numpy layout of tests/state_format.py,
each refusal of a load by one planted damage, an append against the reference's rule (only the blocks from the one
holding the last saved position are written again), a load of another block size, and a save -> load round trip whose
next verify equals the original's bit for bit."""
import os
import struct

import numpy as np
import pytest

import pyoracle as po
import state_format as sf

# a small attention + MoE model whose context spans several 256-position blocks
CFG = dict(hidden=128, vocab=256, n_layers=2, n_experts=8, top_k=2, moe_ff=64, shared_ff=64, n_heads=4, n_kv_heads=2,
           head_dim=32, rope_dim=16, rope_theta=1e4, eps=1e-6, max_ctx=640)
CTX = 600


def _model(kv_int8=0, seed=3, ctx=CTX):
    return po.Model(dict(CFG, kv_int8=kv_int8), seed=seed, ctx=ctx)


def _rows(om):
    c = om.cfg
    kv_row = c["n_kv_heads"] * c["head_dim"]
    rows, scales = [], []
    for l in range(c["n_layers"] + (1 if c.get("mtp") else 0)):   # (an MTP layer's KV after the main layers')
        if c.get("kv_int8"):
            rows.append(om.tensor(po.KV8, l)[0].view(np.int8).reshape(2, c["max_ctx"], kv_row))
            scales.append(om.tensor(po.KVS, l)[0].view(np.float32).reshape(2, c["max_ctx"], c["n_kv_heads"]))
        else:
            rows.append(om.tensor(po.KV, l)[0].view(np.uint16).reshape(2, c["max_ctx"], kv_row))
    return rows, (scales if c.get("kv_int8") else None)


def test_fnv1a_published_vectors():
    """the FNV-1a step against the published 64-bit vectors (from FNV's own offset basis); the reference's files
    start it from state.cpp:68's 1469598103934665603 instead, which the format tests below carry"""
    for text, want in ((b"", 0xCBF29CE484222325), (b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)):
        assert sf.fnv1a(text, sf.FNV_BASIS) == want
        buf = np.frombuffer(text, np.uint8) if text else np.zeros(1, np.uint8)
        assert po.lib.orc_fnv1a(po._ptr(buf), len(text), sf.FNV_BASIS) == want
    assert sf.fnv1a(b"") == sf.REF_BASIS


@pytest.mark.parametrize("kv_int8", [0, 1])
@pytest.mark.parametrize("pos", [0, 1, 255, 256, 257, 600])
def test_save_writes_the_format(tmp_path, kv_int8, pos):
    om = _model(kv_int8)
    om.position = pos
    hidden = po.normal(5, CFG["hidden"])
    meta = dict(pack_print=0x1234_5678_9ABC_DEF0, conv_id=77, extra=-5, rope_delta=3, has_mtp=True, hidden=hidden)
    path = str(tmp_path / "s.geode")
    om.save_state(path, **meta)
    rows, scales = _rows(om)
    want = sf.state_bytes(om.cfg, rows, scales, pos, **meta)
    got = open(path, "rb").read()
    assert len(got) == len(want)
    assert got == want
    assert not os.path.exists(path + ".tmp")


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_round_trip_continues_identically(tmp_path, kv_int8):
    a = _model(kv_int8, ctx=300)
    a.position = 300
    path = str(tmp_path / "s.geode")
    hidden = po.normal(9, CFG["hidden"])
    a.save_state(path, conv_id=5, extra=42, rope_delta=-1, has_mtp=True, hidden=hidden)
    b = _model(kv_int8, ctx=0)   # the same weights, an empty cache
    info = b.load_state(path, has_mtp=True)
    assert (info["conv_id"], info["extra"], info["rope_delta"]) == (5, 42, -1)
    np.testing.assert_array_equal(info["hidden"], hidden)
    assert b.position == 300
    ra, sa = _rows(a)
    rb, sb = _rows(b)
    for l in range(CFG["n_layers"]):
        np.testing.assert_array_equal(ra[l][:, :300], rb[l][:, :300])
        if kv_int8:
            np.testing.assert_array_equal(sa[l][:, :300], sb[l][:, :300])
    toks = np.array([3, 17, 200, 5], np.int32)
    np.testing.assert_array_equal(a.verify(toks), b.verify(toks))


def _planted(path, what):
    buf = bytearray(open(path, "rb").read())
    h = sf.read_header(buf)
    if what == "magic":
        buf[0] ^= 1
    elif what == "version":
        h["version"] = 2
        buf[:sf.HEADER.size] = sf.pack_header(h)[0]
    elif what == "checksum":
        buf[40] ^= 1   # the position's low byte, the checksum left as it was
    elif what == "cut":
        buf = buf[:-1]
    elif what == "interrupted":   # an append cut short: the fixed part's lead gen bumped, the header not yet written
        struct.pack_into("<Q", buf, h["fixed_offset"], h["gen"] + 1)
    elif what == "too_short":
        buf = buf[:10]
    open(path, "wb").write(bytes(buf))


@pytest.mark.parametrize("what,message", [
    ("magic", "not a saved conversation"), ("version", "another version"), ("checksum", "header is damaged"),
    ("cut", "cut short"), ("interrupted", "incomplete"), ("too_short", "too short"),
    ("pack", "another model"), ("format", "another model"), ("mtp_flag", "another model"),
    ("longer", "longer than this context"), ("missing", "cannot open")])
def test_load_refuses(tmp_path, what, message):
    a = _model(0, ctx=300)
    a.position = 300
    path = str(tmp_path / "s.geode")
    a.save_state(path, pack_print=11)
    if what in ("magic", "version", "checksum", "cut", "interrupted", "too_short"):
        _planted(path, what)
    b = _model(1 if what == "format" else 0, ctx=0)
    if what == "longer":
        b = po.Model(dict(CFG, max_ctx=300), seed=3)
    b.position = 7
    kw = dict(pack_print=12 if what == "pack" else 11, has_mtp=what == "mtp_flag")
    with pytest.raises(ValueError, match=message):
        b.load_state(path + ("x" if what == "missing" else ""), **kw)
    assert b.position == 0   # whatever the failure, the conversation is empty after it


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_append_rewrites_from_the_last_saved_block(tmp_path, kv_int8):
    om = _model(kv_int8)
    path = str(tmp_path / "s.geode")
    om.position = 300
    om.save_state(path, conv_id=9)
    rows, scales = _rows(om)
    before = [r.copy() for r in rows]
    # after the save: a row in block 0 (not written again by an append from position 300, whose last row 299 is in
    # block 1) and the row at 299 (written again) change, as an MTP layer rewrites the row before a new prompt
    rows[0][0, 10, :] = rows[0][0, 11, :]
    rows[1][1, 299, :] = rows[1][1, 298, :]
    if kv_int8:
        scales[0][0, 10, :] = 0.5
        scales[1][1, 299, :] = 0.25
    om.position = 600
    om.save_state(path, append=True, conv_id=9)
    got = open(path, "rb").read()
    h = sf.read_header(got)
    assert h["gen"] == 2 and h["position"] == 600
    expect_rows = [r.copy() for r in rows]
    expect_rows[0][0, 10, :] = before[0][0, 10, :]   # block 0 kept from the first save
    expect_scales = None
    if kv_int8:
        expect_scales = [s.copy() for s in scales]
        # the first save wrote the scales as they were then
        expect_scales[0][0, 10, :] = _model(kv_int8).tensor(po.KVS, 0)[0].view(np.float32).reshape(
            2, CFG["max_ctx"], CFG["n_kv_heads"])[0, 10, :]
    want = sf.state_bytes(om.cfg, expect_rows, expect_scales, 600, conv_id=9, gen=2)
    assert got == want
    # another conversation's append writes the file whole
    om.save_state(path, append=True, conv_id=10)
    assert sf.read_header(open(path, "rb").read())["gen"] == 1


def test_load_takes_another_block_size(tmp_path):
    """the reference's load reads any block size a header names (state.cpp:404-455)"""
    om = _model(0)
    rows, _ = _rows(om)
    path = str(tmp_path / "s.geode")
    open(path, "wb").write(sf.state_bytes(om.cfg, rows, None, 333, block=128, conv_id=4))
    b = _model(0, ctx=0)
    assert b.load_state(path)["conv_id"] == 4 and b.position == 333
    rb, _ = _rows(b)
    for l in range(CFG["n_layers"]):
        np.testing.assert_array_equal(rb[l][:, :333], rows[l][:, :333])


def test_hidden_only_with_mtp_and_a_position(tmp_path):
    om = _model(0)
    path = str(tmp_path / "s.geode")
    om.position = 0
    om.save_state(path, has_mtp=True, hidden=np.ones(CFG["hidden"], np.float32))
    assert sf.read_header(open(path, "rb").read())["has_hidden"] == 0
    om.position = 5
    om.save_state(path, has_mtp=False, hidden=np.ones(CFG["hidden"], np.float32))
    assert sf.read_header(open(path, "rb").read())["has_hidden"] == 0
    om.save_state(path, has_mtp=True, hidden=np.ones(CFG["hidden"], np.float32))
    assert sf.read_header(open(path, "rb").read())["has_hidden"] == 1
    assert om.load_state(path, has_mtp=True)["hidden"].tolist() == [1.0] * CFG["hidden"]


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_mtp_layer_kv_in_the_file(tmp_path, kv_int8):
    """an MTP layer's KV goes after the main layers' (model.cpp:351: n_attn counts it), the fingerprint carries its
    flag; a model without one refuses the file"""
    om = po.Model(dict(CFG, kv_int8=kv_int8, mtp=1), seed=3, ctx=CTX)
    hidden = po.normal(7, CFG["hidden"])
    path = str(tmp_path / "s.geode")
    om.save_state(path, pack_print=9, hidden=hidden)
    rows, scales = _rows(om)
    assert len(rows) == CFG["n_layers"] + 1
    want = sf.state_bytes(om.cfg, rows, scales, CTX, pack_print=9, has_mtp=True, hidden=hidden)
    assert open(path, "rb").read() == want
    with pytest.raises(ValueError):
        _model(kv_int8).load_state(path, pack_print=9, has_mtp=True)


# a model of two Gated DeltaNet layers and an attention layer: its states go in the fixed part (each GDN layer's conv
# state, then each one's recurrent state in the reference's strips), its KV only for the attention layer
GDN = dict(CFG, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
           gdn_layers=[1, 0, 1])


def _gdn_model(ctx, seed=3, kv_int8=0):
    return po.Model(dict(GDN, kv_int8=kv_int8), seed=seed, ctx=ctx)


def _gdn_parts(om):
    """(attention layers' rows, scales, GDN layers' (conv, S)) of the oracle model"""
    c = om.cfg
    kv_row = c["n_kv_heads"] * c["head_dim"]
    conv_dim = 2 * c["gdn_k_heads"] * c["gdn_k_dim"] + c["gdn_v_heads"] * c["gdn_v_dim"]
    rows, scales, gdn = [], [], []
    for l in range(c["n_layers"]):
        if c["gdn_layers"][l]:
            gdn.append((om.tensor(po.GDN_CONV_ST, l)[0].view(np.float32).reshape(conv_dim, c["conv_kernel"] - 1),
                        om.tensor(po.GDN_S, l)[0].view(np.float32).reshape(c["gdn_v_heads"], c["gdn_k_dim"],
                                                                           c["gdn_v_dim"])))
        elif c.get("kv_int8"):
            rows.append(om.tensor(po.KV8, l)[0].view(np.int8).reshape(2, c["max_ctx"], kv_row))
            scales.append(om.tensor(po.KVS, l)[0].view(np.float32).reshape(2, c["max_ctx"], c["n_kv_heads"]))
        else:
            rows.append(om.tensor(po.KV, l)[0].view(np.uint16).reshape(2, c["max_ctx"], kv_row))
    return rows, (scales if c.get("kv_int8") else None), gdn


def test_strips_are_the_references_layout():
    """[dv / 16][dk][16] a head: element (i, j) of head h at h dk dv + (j / 16) dk 16 + i 16 + j % 16"""
    S = np.arange(2 * 8 * 32, dtype=np.float32).reshape(2, 8, 32)
    flat = sf.strips(S).reshape(-1)
    for h, i, j in ((0, 0, 0), (0, 3, 17), (1, 7, 31), (1, 5, 2)):
        assert flat[h * 8 * 32 + (j // 16) * 8 * 16 + i * 16 + j % 16] == S[h, i, j]
    np.testing.assert_array_equal(sf.unstrips(flat, 2, 8, 32), S)


@pytest.mark.parametrize("kv_int8", [0, 1])
@pytest.mark.parametrize("pos", [0, 300])
def test_gdn_save_writes_the_format(tmp_path, kv_int8, pos):
    om = _gdn_model(300, kv_int8=kv_int8)
    om.position = pos
    path = str(tmp_path / "s.geode")
    om.save_state(path, pack_print=99, conv_id=3)
    rows, scales, gdn = _gdn_parts(om)
    assert np.abs(gdn[0][1]).max() > 0 and np.abs(gdn[1][0]).max() > 0   # (a conversation's states, not zeros)
    got = open(path, "rb").read()
    want = sf.state_bytes(om.cfg, rows, scales, pos, pack_print=99, conv_id=3, gdn=gdn)
    assert got == want
    h = sf.read_header(got)
    assert h["n_attn"] == 1 and h["conv_n"] == 2 * 256 * 3 and h["gdn_n"] == 2 * 4 * 32 * 32


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_gdn_round_trip_continues_identically(tmp_path, kv_int8):
    a = _gdn_model(300, kv_int8=kv_int8)
    a.position = 300
    path = str(tmp_path / "s.geode")
    a.save_state(path, conv_id=8)
    b = _gdn_model(0, kv_int8=kv_int8)   # the same weights, zero states and an empty cache
    assert b.load_state(path)["conv_id"] == 8 and b.position == 300
    ra, sa, ga = _gdn_parts(a)
    rb, sb, gb = _gdn_parts(b)
    np.testing.assert_array_equal(ra[0][:, :300], rb[0][:, :300])
    for (ca, Sa), (cb, Sb) in zip(ga, gb):
        np.testing.assert_array_equal(ca, cb)
        np.testing.assert_array_equal(Sa, Sb)
    toks = np.array([3, 17, 200, 5], np.int32)
    np.testing.assert_array_equal(a.verify(toks), b.verify(toks))


def test_gdn_refused_load_leaves_zero_states(tmp_path):
    """Model::reset on a refused load (state.cpp:376-380, model.cpp:1918-1925): the GDN states zero, no position"""
    a = _gdn_model(300)
    a.position = 300
    path = str(tmp_path / "s.geode")
    a.save_state(path, pack_print=1)
    b = _gdn_model(300)
    with pytest.raises(ValueError, match="another model"):
        b.load_state(path, pack_print=2)
    assert b.position == 0
    for conv, S in _gdn_parts(b)[2]:
        assert not conv.any() and not S.any()
    # an attention-only model does not take a GDN model's file, nor the other way round
    with pytest.raises(ValueError, match="another model"):
        _model(0, ctx=0).load_state(path, pack_print=1)
