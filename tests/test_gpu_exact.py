"""The exact path on the GPU (gv_model_config.exact = 1; the reference's ModelOptions::exact / GEODE_EXACT=1,
engine/src/model.cpp:3337-3361 with matvec_rows, kernels.cpp:1230-1250: fp32 activations against the dequantized
weights) against the oracle's exact mode (mode 1, which keeps the cache in fp16 as the GPU does): a gated-attention
model, a model with Gated DeltaNet layers and the MTP draft; chain, tree and keep. The products' operands are the fp32
values as hi + lo fp16 halves (to 2^-22), the sums in fp32 in the matrix cores' order, so the logits agree to ~1e-6 of
their scale; asserted within 1e-4, routed experts identical except at near-ties (K-th and (K+1)-th router logits within
1e-4). A model of each mode in one process: the library switches the operands' mode between their calls, so each
model's results are those it gives alone."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, rel_err, route_margins, tree_parents

pytestmark = pytest.mark.gpu

CTX = 90
TOL = 1e-4
GDN = dict(SMALL, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
           gdn_layers=[1, 0, 1])
SHAPES = {"attn": dict(SMALL, mtp=1), "gdn": dict(GDN, mtp=1)}


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module", params=sorted(SHAPES))
def pair(gv, request):
    cfg = SHAPES[request.param]
    om = po.Model(cfg, seed=31, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(dict(cfg, exact=1))
    adopt_oracle_model(gm, om, CTX)
    yield om, gm
    gm.close()


def _step(om, gm, toks, parents=None):
    ol, oids, tr = om.verify_trace(toks, parents, mode=1)
    gl = gm.verify(toks, parents=parents)
    assert rel_err(gl, ol) <= TOL, f"logits {rel_err(gl, ol):.3e}"
    gids = gm.route_ids(len(toks))
    margins = route_margins(om, tr)
    for l, r in np.argwhere((oids != gids).any(axis=2)):
        assert margins[l, r] < TOL, f"experts differ at layer {l} row {r} (router gap {margins[l, r]:.3e})"
    return gl, ol


def test_chain_tree_keep(pair):
    om, gm = pair
    om.position = gm.position = CTX
    _step(om, gm, np.array([5, 99, 300, 7, 41], np.int32))
    om.keep(3)
    gm.keep(3)
    par = tree_parents((4, 3))
    toks = (np.arange(par.size) * 29 + 11).astype(np.int32) % SMALL["vocab"]
    _step(om, gm, toks, par)
    om.keep(3, [0, 2, 9])
    gm.keep(3, [0, 2, 9])
    _step(om, gm, np.array([8, 13, 21, 34], np.int32))


def test_mtp_draft(pair):
    om, gm = pair
    rng = np.random.default_rng(3)
    toks = rng.integers(0, SMALL["vocab"], 4).astype(np.int32)
    hid = rng.normal(0, 1, (4, SMALL["hidden"])).astype(np.float32)
    od, op, ol = om.draft(toks, CTX + 20, hid, mode=1)
    gd, gp = gm.draft(toks, CTX + 20, hid)
    gl = gm.draft_logits()
    assert rel_err(gl, ol) <= TOL
    s = np.sort(ol)
    if s[-1] - s[-2] > 2 * np.abs(gl - ol).max():
        assert gd == od and gp == pytest.approx(op, rel=1e-4)


def test_models_of_both_modes_in_one_process(gv):
    """an int8-path model and an exact one with the same weights, called in turns: each gives what it gives alone"""
    om = po.Model(SMALL, seed=32, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    a = gv.VerifyModel(SMALL)
    b = gv.VerifyModel(dict(SMALL, exact=1))
    try:
        adopt_oracle_model(a, om, CTX)
        adopt_oracle_model(b, om, CTX)
        steps = [np.array([3 + i, 70 + i, 500 - i], np.int32) for i in range(3)]
        alone_a, alone_b = [], []
        for t in steps:
            a.position = CTX
            alone_a.append(a.verify(t))
        for t in steps:
            b.position = CTX
            alone_b.append(b.verify(t))
        for i, t in enumerate(steps):
            a.position = b.position = CTX
            np.testing.assert_array_equal(a.verify(t), alone_a[i])
            np.testing.assert_array_equal(b.verify(t), alone_b[i])
        assert rel_err(alone_b[0], alone_a[0]) > 1e-6   # (the two modes differ)
        om.position = CTX
        assert rel_err(alone_a[-1], om.verify(steps[-1], mode=0)) <= 1e-2
    finally:
        a.close()
        b.close()


def test_exact_refuses_an_int8_cache(gv):
    with pytest.raises(gv.GeodeError):
        gv.VerifyModel(dict(SMALL, exact=1, kv_int8=1))
