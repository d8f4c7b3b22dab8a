"""A geode-pack loaded into the GPU model (gv_model_load_pack) against the same tensors adopted directly: the next
verify is bit-identical (chain and tree), with the experts in rows and in the tile8 layout; a state saved under the
pack's print loads only with it."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, tree_parents
from pack_writer import write_pack

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module")
def om():
    return po.Model(SMALL, seed=21, router_sigma=SMALL_ROUTER_SIGMA, ctx=0)


@pytest.mark.parametrize("tile8", [False, True], ids=["rows", "tile8"])
def test_pack_loads_as_the_direct_adoption(gv, om, tmp_path, tile8):
    write_pack(om, str(tmp_path), tile8=tile8)
    pack = gv.Pack(str(tmp_path))
    cfg = pack.model_config(max_ctx=SMALL["max_ctx"], max_rows=SMALL["max_rows"])
    for k in SMALL:
        assert cfg[k] == (np.float32(SMALL[k]) if isinstance(SMALL[k], float) else SMALL[k]), k
    a = gv.VerifyModel(SMALL)
    adopt_oracle_model(a, om, 0)
    b = gv.VerifyModel(cfg)
    b.load_pack(pack)
    assert b.position == 0
    toks = np.array([3, 77, 410, 9, 200], np.int32)
    np.testing.assert_array_equal(b.verify(toks), a.verify(toks))
    par = tree_parents((4, 3))
    ttoks = (np.arange(par.size) * 37 % SMALL["vocab"]).astype(np.int32)
    np.testing.assert_array_equal(b.verify(ttoks, par), a.verify(ttoks, par))


def test_state_carries_the_pack_print(gv, om, tmp_path):
    write_pack(om, str(tmp_path / "p"))
    pack = gv.Pack(str(tmp_path / "p"))
    m = gv.VerifyModel(pack.model_config(max_ctx=SMALL["max_ctx"]))
    m.load_pack(pack)
    m.verify(np.array([1, 2, 3], np.int32))
    path = str(tmp_path / "s.geode")
    m.save_state(path, pack_print=pack.print)
    with pytest.raises(gv.StateError, match="model fingerprint"):
        m.load_state(path, pack_print=pack.print ^ 1)
    assert m.load_state(path, pack_print=pack.print)["conv_id"] == 0 and m.position == 3


GDN = dict(SMALL, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
           gdn_layers=[1, 0, 1])


@pytest.mark.parametrize("tile8", [False, True], ids=["rows", "tile8"])
def test_gdn_pack_loads_as_the_direct_adoption(gv, tmp_path, tile8):
    """a pack with Gated DeltaNet layers (linear_attn.* tensors, layer_types linear_attention): the config's shape
    and the next verifies (chain, then a tree from the states the chain left) bit-identical to the direct adoption"""
    om = po.Model(GDN, seed=22, router_sigma=SMALL_ROUTER_SIGMA, ctx=0)
    write_pack(om, str(tmp_path), tile8=tile8)
    pack = gv.Pack(str(tmp_path))
    cfg = pack.model_config(max_ctx=GDN["max_ctx"], max_rows=GDN["max_rows"])
    for k in ("gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim", "conv_kernel", "gdn_layers", "n_layers"):
        assert cfg[k] == GDN[k], k
    a = gv.VerifyModel(GDN)
    adopt_oracle_model(a, om, 0)
    b = gv.VerifyModel(cfg)
    b.load_pack(pack)
    toks = np.array([3, 77, 410, 9, 200], np.int32)
    np.testing.assert_array_equal(b.verify(toks), a.verify(toks))
    par = tree_parents((4, 3))
    ttoks = (np.arange(par.size) * 37 % GDN["vocab"]).astype(np.int32)
    np.testing.assert_array_equal(b.verify(ttoks, par), a.verify(ttoks, par))
    for l in (0, 2):
        for x, y in zip(a.gdn_state(l), b.gdn_state(l)):
            np.testing.assert_array_equal(x, y)
    a.close()
    b.close()


@pytest.mark.parametrize("vocab", [None, "draft"], ids=["whole", "draft_vocab"])
def test_mtp_pack_loads_as_the_direct_adoption(gv, tmp_path, vocab):
    """a pack with an MTP layer (mtp.* tensors, the manifest's "mtp" experts) and optionally a draft_vocab.bin (ids
    outside the vocabulary skipped, model.cpp:806-811): the config's mtp flag, and the drafts and their logits after
    a verify bit-identical to the direct adoption with the same draft vocabulary"""
    cfg0 = dict(SMALL, mtp=1)
    om = po.Model(cfg0, seed=23, router_sigma=SMALL_ROUTER_SIGMA, ctx=0)
    ids = None if vocab is None else [5, 300, -1, 17, SMALL["vocab"], 260, 4, 99]
    write_pack(om, str(tmp_path), draft_vocab=ids)
    pack = gv.Pack(str(tmp_path))
    cfg = pack.model_config(max_ctx=SMALL["max_ctx"], max_rows=SMALL["max_rows"])
    assert cfg["mtp"] == 1
    a = gv.VerifyModel(cfg0)
    adopt_oracle_model(a, om, 0)
    if ids is not None:
        a.set_draft_vocab([i for i in ids if 0 <= i < SMALL["vocab"]])
    b = gv.VerifyModel(cfg)
    b.load_pack(pack)
    try:
        toks = np.array([3, 77, 410, 9, 200], np.int32)
        np.testing.assert_array_equal(b.verify(toks), a.verify(toks))
        nxt = np.array([77, 410, 9, 200, 12], np.int32)
        assert a.draft(nxt, 0) == b.draft(nxt, 0)
        np.testing.assert_array_equal(a.draft_logits(), b.draft_logits())
        if ids is not None:
            assert a.draft_logits().size == 6
        d, _ = a.draft(nxt, 0)
        assert a.draft_next(d, 5) == b.draft_next(d, 5)
        np.testing.assert_array_equal(a.draft_logits(), b.draft_logits())
    finally:
        a.close()
        b.close()
