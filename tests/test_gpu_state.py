"""The GPU model's conversation state (gv_model_save_state / gv_model_load_state) against the oracle's and the
format's restatement in tests/state_format.py: a save of the same cache is the same file byte for byte (fp16 and
int8), a state saved by either side loads into the other and the next verify continues bit for bit (GPU -> GPU) or
within the verify tolerance (GPU -> oracle), an append equals a whole save but for its generation, another block size
loads, and damaged files are refused with the reference's error classes and an empty conversation."""
import struct

import numpy as np
import pytest

import pyoracle as po
import state_format as sf
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, rel_err

pytestmark = pytest.mark.gpu

CFG = dict(SMALL, max_ctx=640)
CTX = 600
META = dict(pack_print=0xFEED_5EED, conv_id=123, extra=-1, rope_delta=0, has_mtp=True)


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module", params=[0, 1], ids=["fp16", "int8"])
def pair(gv, request):
    """(oracle model, GPU model holding the oracle's first CTX positions, the config)"""
    cfg = dict(CFG, kv_int8=request.param)
    om = po.Model(cfg, seed=11, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(cfg)
    adopt_oracle_model(gm, om, CTX)
    return om, gm, cfg


def _fresh(gv, om, cfg):
    """a GPU model with the oracle's weights and an empty cache"""
    gm = gv.VerifyModel(cfg)
    adopt_oracle_model(gm, om, 0)
    return gm


@pytest.mark.parametrize("pos", [1, 255, 256, 257, 600])
def test_save_equals_the_oracles(pair, tmp_path, pos):
    om, gm, _ = pair
    hidden = po.normal(3, CFG["hidden"])
    om.position = pos
    gm.position = pos
    om.save_state(str(tmp_path / "o.geode"), hidden=hidden, **META)
    gm.save_state(str(tmp_path / "g.geode"), hidden=hidden, **META)
    want = open(tmp_path / "o.geode", "rb").read()
    got = open(tmp_path / "g.geode", "rb").read()
    assert len(got) == len(want)
    assert got == want


def test_oracle_state_loads_and_continues(gv, pair, tmp_path):
    om, gm, cfg = pair
    om.position = 555
    om.save_state(str(tmp_path / "o.geode"), **META)
    g2 = _fresh(gv, om, cfg)
    info = g2.load_state(str(tmp_path / "o.geode"), pack_print=META["pack_print"], has_mtp=True)
    assert (info["conv_id"], info["extra"], g2.position) == (123, -1, 555)
    gm.position = 555
    toks = np.array([5, 9, 300, 2, 77], np.int32)
    np.testing.assert_array_equal(g2.verify(toks), gm.verify(toks))


def test_state_after_gpu_steps_round_trips(gv, pair, tmp_path):
    """KV rows the GPU's own steps appended (across the 256-position block edge) survive a save and a load: the next
    verify is bit-identical on the GPU and within the verify tolerance on the oracle"""
    om, _, cfg = pair
    gm = gv.VerifyModel(cfg)   # its own model: the steps overwrite cache rows the other tests compare
    adopt_oracle_model(gm, om, 250)
    rng = np.random.default_rng(4)
    for _ in range(3):
        gm.verify(rng.integers(0, cfg["vocab"], 5).astype(np.int32))
        gm.keep(4)
    assert gm.position == 262
    path = str(tmp_path / "g.geode")
    gm.save_state(path, **META)
    g2 = _fresh(gv, om, cfg)
    g2.load_state(path, pack_print=META["pack_print"], has_mtp=True)
    toks = np.array([1, 2, 3], np.int32)
    want = gm.verify(toks)
    np.testing.assert_array_equal(g2.verify(toks), want)
    o2 = po.Model(cfg, seed=11, router_sigma=SMALL_ROUTER_SIGMA, ctx=0)
    o2.load_state(path, pack_print=META["pack_print"], has_mtp=True)
    assert o2.position == 262
    err = rel_err(want, o2.verify(toks))
    assert err <= 1e-2, f"logits max error {err:.3e}"


def _with_gen(buf, gen):
    """a whole save's bytes as an append of generation gen writes them"""
    b = bytearray(buf)
    h = sf.read_header(b)
    lo = sf.layout(h)
    h["gen"] = gen
    b[:sf.HEADER.size] = sf.pack_header(h)[0]
    struct.pack_into("<Q", b, h["fixed_offset"], gen)
    struct.pack_into("<Q", b, lo["trail"], gen)
    return bytes(b)


def test_append_equals_a_whole_save(pair, tmp_path):
    om, gm, _ = pair
    path = str(tmp_path / "a.geode")
    gm.position = 300
    gm.save_state(path, **META)
    gm.position = 590
    gm.save_state(path, append=True, **META)
    gm.save_state(str(tmp_path / "w.geode"), **META)
    assert open(path, "rb").read() == _with_gen(open(tmp_path / "w.geode", "rb").read(), 2)


def test_another_block_size_loads(gv, pair, tmp_path):
    om, gm, cfg = pair
    kv_row = cfg["n_kv_heads"] * cfg["head_dim"]
    rows, scales = [], None
    for l in range(cfg["n_layers"]):
        if cfg["kv_int8"]:
            rows.append(om.tensor(po.KV8, l)[0].view(np.int8).reshape(2, cfg["max_ctx"], kv_row))
        else:
            rows.append(om.tensor(po.KV, l)[0].view(np.uint16).reshape(2, cfg["max_ctx"], kv_row))
    if cfg["kv_int8"]:
        scales = [om.tensor(po.KVS, l)[0].view(np.float32).reshape(2, cfg["max_ctx"], cfg["n_kv_heads"])
                  for l in range(cfg["n_layers"])]
    path = str(tmp_path / "b.geode")
    open(path, "wb").write(sf.state_bytes(cfg, rows, scales, 333, block=128, conv_id=8))
    g2 = _fresh(gv, om, cfg)
    assert g2.load_state(path)["conv_id"] == 8 and g2.position == 333
    gm.position = 333
    toks = np.array([40, 41], np.int32)
    np.testing.assert_array_equal(g2.verify(toks), gm.verify(toks))


@pytest.mark.parametrize("what,kind", [("checksum", "format"), ("interrupted", "io"), ("cut", "io"),
                                       ("pack", "format"), ("longer", "arg")])
def test_damaged_files_are_refused(gv, pair, tmp_path, what, kind):
    om, gm, cfg = pair
    path = str(tmp_path / "d.geode")
    gm.position = 300
    gm.save_state(path, **META)
    buf = bytearray(open(path, "rb").read())
    h = sf.read_header(buf)
    if what == "checksum":
        buf[40] ^= 1
    elif what == "interrupted":
        struct.pack_into("<Q", buf, h["fixed_offset"], h["gen"] + 1)
    elif what == "cut":
        buf = buf[:-1]
    open(path, "wb").write(bytes(buf))
    g2 = gv.VerifyModel(dict(cfg, max_ctx=300)) if what == "longer" else _fresh(gv, om, cfg)
    if what == "longer":
        adopt_oracle_model(g2, om, 0)
    g2.position = 5
    with pytest.raises(gv.StateError) as e:
        g2.load_state(path, pack_print=META["pack_print"] + (what == "pack"), has_mtp=True)
    assert e.value.kind == kind
    assert g2.position == 0


# a model of Gated DeltaNet layers around an attention layer (its states in the file's fixed part)
GDN_CFG = dict(CFG, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
               gdn_layers=[1, 0, 1])


@pytest.fixture(scope="module", params=[0, 1], ids=["fp16", "int8"])
def gdn_pair(gv, request):
    cfg = dict(GDN_CFG, kv_int8=request.param)
    om = po.Model(cfg, seed=12, router_sigma=SMALL_ROUTER_SIGMA, ctx=300)
    gm = gv.VerifyModel(cfg)
    adopt_oracle_model(gm, om, 300)
    yield om, gm, cfg
    gm.close()


@pytest.mark.parametrize("pos", [0, 300])
def test_gdn_save_equals_the_oracles(gdn_pair, tmp_path, pos):
    """the same states and cache (adopted, no step since): the same file byte for byte"""
    om, gm, _ = gdn_pair
    om.position = pos
    gm.position = pos
    om.save_state(str(tmp_path / "o.geode"), **META)
    gm.save_state(str(tmp_path / "g.geode"), **META)
    assert open(tmp_path / "g.geode", "rb").read() == open(tmp_path / "o.geode", "rb").read()


def test_gdn_state_round_trips_and_continues(gv, gdn_pair, tmp_path):
    """a GPU save after a verify and keep (the states of the kept row) loads into a fresh GPU model: its states the
    same, and the next verify the same bit for bit"""
    om, gm, cfg = gdn_pair
    gm.position = 300
    gm.verify(np.array([4, 8, 15, 16, 23], np.int32))
    gm.keep(3)
    path = str(tmp_path / "g.geode")
    gm.save_state(path, **META)
    g2 = gv.VerifyModel(cfg)
    adopt_oracle_model(g2, om, 0)
    assert g2.load_state(path, pack_print=META["pack_print"], has_mtp=True)["conv_id"] == 123
    assert g2.position == 303
    for l in (0, 2):
        for a, b in zip(gm.gdn_state(l), g2.gdn_state(l)):
            np.testing.assert_array_equal(a, b)
    toks = np.array([42, 7, 99], np.int32)
    np.testing.assert_array_equal(g2.verify(toks), gm.verify(toks))
    # the file's states read by the format's restatement are the model's
    buf = open(path, "rb").read()
    for (conv, S), l in zip(sf.gdn_states(cfg, buf), (0, 2)):
        g2.position = 303
        g2.load_state(path, pack_print=META["pack_print"], has_mtp=True)
        gc, gs = g2.gdn_state(l)
        np.testing.assert_array_equal(conv, gc)
        np.testing.assert_array_equal(S, gs)
    g2.close()


def test_gdn_refused_load_leaves_zero_states(gv, gdn_pair, tmp_path):
    om, gm, cfg = gdn_pair
    gm.position = 300
    path = str(tmp_path / "g.geode")
    gm.save_state(path, **META)
    g2 = gv.VerifyModel(cfg)
    adopt_oracle_model(g2, om, 300)
    with pytest.raises(gv.StateError):
        g2.load_state(path, pack_print=META["pack_print"] + 1, has_mtp=True)
    assert g2.position == 0
    for l in (0, 2):
        conv, S = g2.gdn_state(l)
        assert not conv.any() and not S.any()
    g2.close()


@pytest.mark.parametrize("kv_int8", [0, 1])
def test_mtp_save_equals_the_oracles(gv, tmp_path, kv_int8):
    """a model with an MTP layer: its KV after the main layers' in every block (model.cpp:351), the fingerprint's MTP
    flag from the model; the GPU's file equals the oracle's byte for byte after an MTP pass on both, and it loads into a
    fresh GPU model whose next draft equals the original's"""
    cfg = dict(CFG, kv_int8=kv_int8, mtp=1, max_ctx=400)
    om = po.Model(cfg, seed=13, router_sigma=SMALL_ROUTER_SIGMA, ctx=300)
    gm = gv.VerifyModel(cfg)
    g2 = None
    try:
        adopt_oracle_model(gm, om, 300)
        rng = np.random.default_rng(4)
        toks = rng.integers(0, cfg["vocab"], 3).astype(np.int32)
        hid = rng.normal(0, 1, (3, cfg["hidden"])).astype(np.float32)
        om.mtp(toks, 280, hid, logits=False)
        gm.mtp_fill(toks, 280, hid)
        om.position = gm.position = 300
        meta = dict(META, has_mtp=False)   # (the model's own MTP layer sets the flag)
        om.save_state(str(tmp_path / "o.geode"), **meta)
        gm.save_state(str(tmp_path / "g.geode"), **meta)
        got, want = open(tmp_path / "g.geode", "rb").read(), open(tmp_path / "o.geode", "rb").read()
        assert len(got) == len(want) and got[:4096] == want[:4096]   # the header: n_attn 3, the MTP flag
        assert sf.read_header(got)["n_attn"] == cfg["n_layers"] + 1
        # the KV blocks: every row equal but the MTP pass's own (positions 280..282 of the MTP layer's, where the
        # two paths' products may differ in the last bits)
        gr, gs = sf.kv_rows(cfg, got)
        orr, os_ = sf.kv_rows(cfg, want)
        for l in range(cfg["n_layers"] + 1):
            live = np.ones(300, bool)
            if l == cfg["n_layers"]:
                live[280:283] = False
            assert np.array_equal(gr[l][:, live], orr[l][:, live]), f"attention layer {l}"
            if kv_int8:
                assert np.array_equal(gs[l][:, live], os_[l][:, live])
        g2 = _fresh(gv, om, cfg)
        g2.load_state(str(tmp_path / "g.geode"), pack_print=meta["pack_print"])
        t2 = np.array([5, 6], np.int32)
        h2 = rng.normal(0, 1, (2, cfg["hidden"])).astype(np.float32)
        a = gm.draft(t2, 300, h2)
        la = gm.draft_logits()
        b = g2.draft(t2, 300, h2)
        assert a == b and np.array_equal(la, g2.draft_logits())
    finally:
        gm.close()
        if g2 is not None:
            g2.close()
