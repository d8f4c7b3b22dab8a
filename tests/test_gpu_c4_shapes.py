"""GPU parity at the configs' own shapes (BASELINE.json configs[2] and [3]): hidden 2048, 16 query heads and 2 KV heads
of 256 (RoPE on 64 dims), 256 experts + 1 shared of ff 512, top-8 routing; one layer, a 1,024-token vocabulary and a
300-position context keep the oracle quick. The weights are the oracle's seeded random q4 bytes (valid codes and
finite E4M3 scales, not packed from floats: the arithmetic is what is compared). Against the oracle's int8 path:
logits and MoE outputs within 1e-2 (max error over max |value|), routed experts identical; chain (M = 5) and the
16-node draft tree (M = 17), whose many experts a step exercise every slot of the decode MoE."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import adopt_oracle_model, near_tie_rows, rel_err, tree_parents

pytestmark = pytest.mark.gpu

C4_1L = dict(hidden=2048, vocab=1024, n_layers=1, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
             n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=400, max_rows=17)
CTX = 300


@pytest.fixture(scope="module")
def models():
    import geode_amd

    geode_amd.init(0)
    om = po.Model(C4_1L, seed=5, router_sigma=1.0 / np.sqrt(C4_1L["hidden"]), ctx=CTX, fast=True)
    gm = geode_amd.VerifyModel(C4_1L)
    adopt_oracle_model(gm, om, CTX)
    yield om, gm
    gm.close()


def _check(ol, gl, oids, gids):
    err = rel_err(gl, ol)
    assert err <= 1e-2, f"logits max error {err:.3e}"
    assert np.array_equal(oids, gids), f"routing agrees on {np.mean(oids == gids):.4f} of picks"
    ties = near_tie_rows(ol, 2 * np.abs(gl - ol).max())
    for r in range(ol.shape[0]):
        if r not in ties:
            assert np.argmax(gl[r]) == np.argmax(ol[r]), f"greedy token differs at row {r}"


@pytest.mark.parametrize("tree", [False, True])
def test_verify_step(models, tree):
    om, gm = models
    parents = tree_parents((4, 3)) if tree else None
    n = 17 if tree else 5
    toks = (np.arange(n) * 131 + 17) % C4_1L["vocab"]
    om.position = CTX
    gm.position = CTX
    ol, oids = om.verify(toks, parents, route=True)
    gl = gm.verify(toks, parents=parents)
    _check(ol, gl, oids, gm.route_ids(n))


@pytest.mark.parametrize("M", [5, 17])
def test_moe_block(models, M):
    """one MoE block, fp16-valued rows N(0, 1), routed logits N(0, 1) given"""
    om, gm = models
    H, E = C4_1L["hidden"], C4_1L["n_experts"]
    h = np.array([po.lib.orc_f16_to_f32(po.lib.orc_f32_to_f16(float(v))) for v in po.normal(31 + M, M * H, 1.0)],
                 np.float32).reshape(M, H)
    lg = po.normal(32 + M, M * E, 1.0).reshape(M, E)
    want, wids, wwts = po.moe_layer(om, 0, h, lg)
    got, gids, gwts = gm.moe(0, h, lg)
    assert np.array_equal(gids, wids)
    assert np.abs(gwts - wwts).max() <= 1e-6
    assert rel_err(got, want) <= 1e-2, f"max error {rel_err(got, want):.3e}"


def test_repeated_steps_identical(models):
    """the same step many times (graph replays after the first two): the same bits every time"""
    om, gm = models
    toks = np.array([101, 202, 303, 404, 505], np.int32)
    gm.position = CTX
    first = gm.verify(toks)
    for _ in range(6):
        gm.position = CTX
        again = gm.verify(toks)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32))


@pytest.mark.parametrize("level", [1, 2])
@pytest.mark.parametrize("tree", [False, True])
def test_fused_launches_match_separate_kernels(models, tree, level):
    """the dependent phases chained within one launch (the default where the shapes fit; level 1: the rows routed by
    the experts' up launch, 2: by the output projection's launch) against one launch a phase: the same arithmetic in
    the same order, so the same bits; several steps in a row (graph replays after the second)"""
    om, gm = models
    parents = tree_parents((4, 3)) if tree else None
    n = 17 if tree else 5
    toks = (np.arange(n) * 211 + 9) % C4_1L["vocab"]
    gm.set_fused(False)
    gm.position = CTX
    want = gm.verify(toks, parents=parents)
    want_ids = gm.route_ids(n)
    gm.set_fused(level)
    try:
        for _ in range(5):
            gm.position = CTX
            got = gm.verify(toks, parents=parents)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            assert np.array_equal(gm.route_ids(n), want_ids)
    finally:
        gm.set_fused(True)
