"""GPU parity of the int8 KV cache (config kv_int8; attend<int8_t>, engine/src/model.cpp:3756-3792, :3929-3972)
against the oracle's int8 path on the same seeded weights and context: the small model (head_dim 64) and the
configs' attention shape (head_dim 256, one layer); chain and tree, logits within 1e-2 (max error over max |logit|)
and routed experts identical; a tree's kept path compacted in the int8 cache (values and scales) as the oracle
compacts it."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, near_tie_rows, rel_err, tree_parents

pytestmark = pytest.mark.gpu

CTX = 100
SMALL8 = dict(SMALL, kv_int8=1)
C4_1L8 = dict(hidden=2048, vocab=1024, n_layers=1, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
              n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=400, max_rows=17, kv_int8=1)


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module")
def small(gv):
    om = po.Model(SMALL8, seed=7, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(SMALL8)
    adopt_oracle_model(gm, om, CTX)
    yield om, gm
    gm.close()


@pytest.fixture(scope="module")
def c4(gv):
    ctx = 300
    om = po.Model(C4_1L8, seed=5, router_sigma=1.0 / np.sqrt(C4_1L8["hidden"]), ctx=ctx, fast=True)
    gm = gv.VerifyModel(C4_1L8)
    adopt_oracle_model(gm, om, ctx)
    yield om, gm, ctx
    gm.close()


def _check(ol, gl, oids, gids):
    err = rel_err(gl, ol)
    assert err <= 1e-2, f"logits max error {err:.3e}"
    assert np.array_equal(oids, gids), f"routing agrees on {np.mean(oids == gids):.4f} of picks"
    ties = near_tie_rows(ol, 2 * np.abs(gl - ol).max())
    for r in range(ol.shape[0]):
        if r not in ties:
            assert np.argmax(gl[r]) == np.argmax(ol[r]), f"greedy token differs at row {r}"


@pytest.mark.parametrize("n", [1, 2, 5])
def test_chain(small, n):
    om, gm = small
    toks = (np.arange(n) * 97 + 13) % SMALL["vocab"]
    om.position = CTX
    gm.position = CTX
    ol, oids = om.verify(toks, route=True)
    gl = gm.verify(toks)
    _check(ol, gl, oids, gm.route_ids(n))


def test_tree(small):
    om, gm = small
    parents = tree_parents((4, 3))
    toks = (np.arange(parents.size) * 31 + 7) % SMALL["vocab"]
    om.position = CTX
    gm.position = CTX
    ol, oids = om.verify(toks, parents, route=True)
    gl = gm.verify(toks, parents=parents)
    _check(ol, gl, oids, gm.route_ids(parents.size))


def test_tree_keep_compacts_the_int8_cache(small):
    om, gm = small
    parents = tree_parents((4, 3))
    toks = (np.arange(parents.size) * 53 + 5) % SMALL["vocab"]
    path = np.array([0, 3, 11], np.int32)   # row 11 is a child of row 3
    for m in (om, gm):
        m.position = CTX
        m.verify(toks, parents)
        m.keep(3, path)
    nxt = np.array([77, 78], np.int32)
    ol, oids = om.verify(nxt, route=True)
    gl = gm.verify(nxt)
    _check(ol, gl, oids, gm.route_ids(2))


@pytest.mark.parametrize("tree", [False, True])
def test_c4_shape(c4, tree):
    om, gm, ctx = c4
    parents = tree_parents((4, 3)) if tree else None
    n = 17 if tree else 5
    toks = (np.arange(n) * 131 + 17) % C4_1L8["vocab"]
    om.position = ctx
    gm.position = ctx
    ol, oids = om.verify(toks, parents, route=True)
    gl = gm.verify(toks, parents=parents)
    _check(ol, gl, oids, gm.route_ids(n))
