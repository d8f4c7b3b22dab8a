"""GPU parity of the whole verify step (C4's family at small shapes) against the oracle on the same seeded inputs:
logits within 1e-2 (max error over max |logit|) of the reference's default int8 CPU path, routed experts
identical, greedy tokens identical away from near-ties; chain and tree; verify + keep equal to a verify of the kept
prefix."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, near_tie_rows, rel_err, tree_parents

pytestmark = pytest.mark.gpu

CTX = 100


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module")
def models(gv):
    om = po.Model(SMALL, seed=7, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(SMALL)
    adopt_oracle_model(gm, om, CTX)
    return om, gm


def _check(om_logits, gm_logits, om_ids, gm_ids):
    err = rel_err(gm_logits, om_logits)
    assert err <= 1e-2, f"logits max error {err:.3e}"
    same_route = np.mean(om_ids == gm_ids)
    assert same_route == 1.0, f"routing agrees on {same_route:.4f} of picks"
    ties = near_tie_rows(om_logits, 2 * np.abs(gm_logits - om_logits).max())
    for r in range(om_logits.shape[0]):
        if r not in ties:
            assert np.argmax(gm_logits[r]) == np.argmax(om_logits[r]), f"greedy token differs at row {r}"


@pytest.mark.parametrize("n", [1, 2, 5])
def test_chain_verify(models, n):
    om, gm = models
    om.position = CTX
    gm.position = CTX
    toks = (np.arange(n) * 37 + 11) % SMALL["vocab"]
    ol, oids = om.verify(toks, route=True)
    gl = gm.verify(toks)
    _check(ol, gl, oids, gm.route_ids(n))


def test_tree_verify(models):
    om, gm = models
    parents = tree_parents((4, 3))   # 17 rows: the root, 4 children, 12 grandchildren
    n = parents.size
    toks = (np.arange(n) * 53 + 5) % SMALL["vocab"]
    om.position = CTX
    gm.position = CTX
    ol, oids = om.verify(toks, parents=parents, route=True)
    gl = gm.verify(toks, parents=parents)
    _check(ol, gl, oids, gm.route_ids(n))


def test_tree_row_equals_chain_of_its_ancestors(models):
    """a tree row's logits equal those of the chain through its ancestors (same positions): on the GPU"""
    _, gm = models
    parents = tree_parents((4, 3))
    toks = (np.arange(parents.size) * 53 + 5) % SMALL["vocab"]
    gm.position = CTX
    tl = gm.verify(toks, parents=parents)
    for node in (1, 4, 5, 16):
        path = [node]
        while parents[path[-1]] >= 0:
            path.append(int(parents[path[-1]]))
        path = path[::-1]
        gm.position = CTX
        cl = gm.verify(toks[path])
        assert rel_err(tl[node], cl[-1]) <= 1e-5


def test_keep_then_verify(models):
    """verify 5, keep 2, verify 3 more == verify the 2 kept + the 3 new at once (oracle and GPU agree throughout)"""
    om, gm = models
    toks = np.array([3, 99, 200, 7, 401], np.int32)
    nxt = np.array([45, 46, 47], np.int32)
    for m in (om, gm):
        m.position = CTX
    om.verify(toks)
    gm.verify(toks)
    om.keep(2)
    gm.keep(2)
    assert gm.position == CTX + 2
    ol = om.verify(nxt)
    gl = gm.verify(nxt)
    assert rel_err(gl, ol) <= 1e-2
    gm.position = CTX
    whole = gm.verify(np.concatenate([toks[:2], nxt]))
    assert rel_err(gl, whole[2:]) <= 1e-5


def test_tree_keep_compacts_kv(models):
    om, gm = models
    parents = tree_parents((4, 3))
    toks = (np.arange(parents.size) * 29 + 1) % SMALL["vocab"]
    path = np.array([0, 2, 9], np.int32)   # root -> its 2nd child -> a grandchild under it
    assert parents[2] == 0 and parents[9] == 2
    for m in (om, gm):
        m.position = CTX
        m.verify(toks, parents=parents)
        m.keep(3, path)
    nxt = np.array([17, 18], np.int32)
    ol = om.verify(nxt)
    gl = gm.verify(nxt)
    assert rel_err(gl, ol) <= 1e-2
    gm.position = CTX
    chain = gm.verify(np.concatenate([toks[path], nxt]))
    assert rel_err(gl, chain[3:]) <= 1e-5


@pytest.mark.parametrize("M,given", [(5, True), (17, True), (5, False)])
def test_moe_block(models, M, given):
    """C3: one MoE block on fp16-valued rows (routed logits given as N(0, 1), or the layer's router): the block's
    output within 1e-2 of the oracle's int8 path (max error over max |out|), the routed experts and weights"""
    om, gm = models
    E = SMALL["n_experts"]
    h = np.array([po.lib.orc_f16_to_f32(po.lib.orc_f32_to_f16(float(v))) for v in po.normal(91 + M, M * SMALL["hidden"], 1.0)],
                 np.float32).reshape(M, SMALL["hidden"])
    lg = po.normal(92 + M, M * E, 1.0).reshape(M, E) if given else None
    want, wids, wwts = po.moe_layer(om, 1, h, lg)
    got, gids, gwts = gm.moe(1, h, lg)
    assert np.array_equal(gids, wids)
    assert np.abs(gwts - wwts).max() <= 1e-6
    assert rel_err(got, want) <= 1e-2, f"max error {rel_err(got, want):.3e}"
    # and the verify state still works afterwards
    om.position = CTX
    gm.position = CTX
    toks = np.array([3, 4], np.int32)
    ol, oids = om.verify(toks, route=True)
    _check(ol, gm.verify(toks), oids, gm.route_ids(2))


@pytest.mark.parametrize("M", [100, 600])
def test_moe_prefill(models, M):
    """C5's path: many rows (more than the verify step's), the routed logits given; experts grouped by expert in runs
    of at most 32 rows (M = 600 gives each of the 16 experts ~150 rows): the block's output within 1e-2 of the
    oracle's int8 path, the routed experts and weights identical"""
    om, gm = models
    E = SMALL["n_experts"]
    h = po.normal(93 + M, M * SMALL["hidden"], 1.0).reshape(M, SMALL["hidden"])
    lg = po.normal(94 + M, M * E, 1.0).reshape(M, E)
    want, wids, wwts = po.moe_layer(om, 0, h, lg)
    got, gids, gwts = gm.moe(0, h, lg)
    assert np.array_equal(gids, wids)
    assert np.abs(gwts - wwts).max() <= 1e-6
    assert rel_err(got, want) <= 1e-2, f"max error {rel_err(got, want):.3e}"


def test_graph_replays_match_direct_launches(models):
    """the step's HIP graph (captured on the second step of a row count) replayed several times, with direct steps
    and other row counts in between: every replay's logits and routing equal the direct launches' bit for bit"""
    om, gm = models
    toks = np.array([21, 22, 23, 24, 25], np.int32)

    def step(n, graphs):
        gm.set_graphs(graphs)
        gm.position = CTX
        lg = gm.verify(toks[:n])
        return lg, gm.route_ids(n)

    want, wids = step(5, False)
    for rep in range(4):
        got, ids = step(5, True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
        assert np.array_equal(ids, wids)
        other, _ = step(2, rep % 2 == 0)   # another row count, graphs on and off, between the replays
        assert np.array_equal(other.view(np.uint32), step(2, False)[0].view(np.uint32))
    gm.set_graphs(True)


@pytest.mark.parametrize("hd,rope", [(96, 32), (32, 16), (160, 64)])
def test_head_dims_off_the_64_grid(gv, hd, rope):
    """head sizes whose 16-dim value tiles are not a multiple of four (the attention's output loop takes them in
    fours): chain and tree against the oracle"""
    cfg = dict(SMALL, head_dim=hd, rope_dim=rope, n_heads=4 if hd % 32 == 0 and (4 * hd) % 128 == 0 else 8)
    om = po.Model(cfg, seed=13, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(cfg)
    try:
        adopt_oracle_model(gm, om, CTX)
        for parents, n in ((None, 5), (tree_parents((4, 3)), 17)):
            toks = (np.arange(n) * 29 + 3) % cfg["vocab"]
            om.position = CTX
            gm.position = CTX
            ol, oids = om.verify(toks, parents, route=True)
            gl = gm.verify(toks, parents=parents)
            _check(ol, gl, oids, gm.route_ids(n))
    finally:
        gm.close()


def test_route_ties_go_to_the_lower_index(models):
    """the GPU route (route_kernel through the MoE block entry point) on router logits with exact ties: the lower
    expert index ranks first, as the oracle's route_topk and the reference's GPU route (gpu8_kernels.inc:974-978)"""
    om, gm = models
    E, K, H = SMALL["n_experts"], SMALL["top_k"], SMALL["hidden"]
    M = 6
    lg = np.zeros((M, E), np.float32)
    lg[0, [2, 9, 11, 14, 15]] = 1.5            # five equal maxima for four picks
    lg[1, :] = 0.25                            # every logit equal
    lg[2, [0, 15]] = 3.0; lg[2, [4, 5, 6]] = 2.0
    lg[3] = np.repeat(np.arange(E // 2, dtype=np.float32), 2)[::-1]   # pairs of equal values
    lg[4, [7, 8]] = -1.0
    lg[5] = po.normal(77, E, 1.0)
    lg[5, 3] = lg[5, 12] = lg[5].max()
    h = po.normal(78, M * H, 1.0).reshape(M, H)
    _, gids, gw = gm.moe(0, h, lg)
    for t in range(M):
        ids, w = po.route_topk(lg[t], K)
        assert list(gids[t]) == list(ids), (t, list(gids[t]), list(ids))
        assert np.abs(gw[t] - w).max() <= 1e-6
