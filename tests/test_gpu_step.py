"""The verify step as one persistent kernel (step.hip) against the per-phase kernels (model.hip) and the oracle.

The persistent kernel does the per-phase kernels' arithmetic operation for operation, so on the same model and rows
both give the same logits, routing and KV cache bit for bit; a stale read of data another workgroup wrote in the
same launch (the kernel's phases exchange everything through device-coherent loads and stores) would show as a
difference. Both shapes families are covered: the tests' small model (every product one or two ranges) and the
configs' 35B-A3B shapes (hidden 2048, 16 x 256 heads, ff 512, 256 experts, vocab 151,936) with a full 8,192-position
context, two layers of them.
"""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, adopt_oracle_model, rel_err, tree_parents

pytestmark = pytest.mark.gpu

CTX = 100


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module")
def small(gv):
    om = po.Model(SMALL, seed=11, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    gm = gv.VerifyModel(SMALL)
    adopt_oracle_model(gm, om, CTX)
    return om, gm


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _step(gm, toks, parents=None, step_kernel=True, pos=CTX):
    gm.set_step_kernel(step_kernel)
    gm.position = pos
    lg = gm.verify(toks, parents=parents)
    return lg, gm.route_ids(len(toks))


@pytest.mark.parametrize("n", [1, 2, 5, 16])
def test_small_chain_matches_kernels(small, n):
    _, gm = small
    assert gm.step_kernel_supported(n)
    toks = (np.arange(n) * 41 + 3) % SMALL["vocab"]
    want, wids = _step(gm, toks, step_kernel=False)
    got, ids = _step(gm, toks, step_kernel=True)
    assert np.array_equal(ids, wids)
    assert np.array_equal(_bits(got), _bits(want)), f"max diff {np.abs(got - want).max():.3e}"


def test_small_tree_matches_kernels(small):
    _, gm = small
    parents = tree_parents((4, 3))
    toks = (np.arange(parents.size) * 53 + 5) % SMALL["vocab"]
    assert gm.step_kernel_supported(parents.size)
    want, wids = _step(gm, toks, parents, step_kernel=False)
    got, ids = _step(gm, toks, parents, step_kernel=True)
    assert np.array_equal(ids, wids)
    assert np.array_equal(_bits(got), _bits(want)), f"max diff {np.abs(got - want).max():.3e}"


def test_small_oracle_parity(small):
    """the persistent kernel against the oracle's int8 path: logits within 1e-2, routing identical"""
    om, gm = small
    toks = np.array([17, 230, 4, 91, 300], np.int32)
    om.position = CTX
    ol, oids = om.verify(toks, route=True)
    gl, gids = _step(gm, toks, step_kernel=True)
    assert rel_err(gl, ol) <= 1e-2
    assert np.array_equal(gids, oids)


def test_small_sequence_with_keep(small):
    """several steps with keeps in between (the KV cache the kernel appends is read by the next step): the same
    logits as the per-phase kernels at every step"""
    _, gm = small
    seqs = [np.array([5, 6, 7, 8, 9], np.int32), np.array([10, 11, 12], np.int32), np.array([13, 14, 15, 16, 17], np.int32)]
    keeps = [3, 2, 5]
    out = {}
    for sk in (False, True):
        gm.set_step_kernel(sk)
        gm.position = CTX
        res = []
        for toks, kept in zip(seqs, keeps):
            res.append(gm.verify(toks))
            gm.keep(kept)
        out[sk] = res
    for a, b in zip(out[False], out[True]):
        assert np.array_equal(_bits(a), _bits(b))


C4_2L = dict(hidden=2048, vocab=151936, n_layers=2, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
             n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=8192 + 64, max_rows=17)
C4_CTX = 8192


@pytest.fixture(scope="module")
def c4(gv):
    gm = gv.VerifyModel(C4_2L)
    gm.randomize(20261201, 0.02, 0.0221, C4_CTX)
    return gm


@pytest.mark.parametrize("n,tree", [(5, False), (1, False), (17, True)])
def test_c4_shapes_match_kernels(c4, n, tree):
    gm = c4
    parents = tree_parents((4, 3)) if tree else None
    assert gm.step_kernel_supported(n)
    toks = (np.arange(n) * 7919 + 13) % C4_2L["vocab"]
    want, wids = _step(gm, toks, parents, step_kernel=False, pos=C4_CTX)
    got, ids = _step(gm, toks, parents, step_kernel=True, pos=C4_CTX)
    assert np.array_equal(ids, wids)
    assert np.array_equal(_bits(got), _bits(want)), f"max diff {np.abs(got - want).max():.3e}"


@pytest.mark.parametrize("toks,pos", [([9500], C4_CTX), ([7, 1007, 2007, 3007, 4007], C4_CTX),
                                      ([7, 1007, 2007, 3007, 4007], 1000)])
def test_c4_key_rounding_cases(c4, toks, pos):
    """token and position sets whose new keys have an element where one rounding of the normalized product to
    fp16 differs from two (fp32, then fp16): both paths must round twice, the cache and logits then agree"""
    gm = c4
    toks = np.array(toks, np.int32)
    want, wids = _step(gm, toks, step_kernel=False, pos=pos)
    got, ids = _step(gm, toks, step_kernel=True, pos=pos)
    assert np.array_equal(ids, wids)
    assert np.array_equal(_bits(got), _bits(want)), f"max diff {np.abs(got - want).max():.3e}"


def test_c4_repeated_steps_stable(c4):
    """the same step eight times through the persistent kernel: the same bits every time"""
    gm = c4
    toks = np.array([101, 202, 303, 404, 505], np.int32)
    first, _ = _step(gm, toks, step_kernel=True, pos=C4_CTX)
    for _ in range(7):
        again, _ = _step(gm, toks, step_kernel=True, pos=C4_CTX)
        assert np.array_equal(_bits(again), _bits(first))
