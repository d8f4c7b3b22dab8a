"""The oracle's Gated DeltaNet layer (oracle/oracle_layers.cpp gdn_layer, a restatement of engine/src/model.cpp:
3497-3688) pinned on the CPU: a model of two GDN layers and an attention layer against the float64 restatement in
tests/f64_model.py (both arithmetic modes, chain and tree), eight planted slips of the GDN composition each caught;
the delta rule alone against its defining property (with decay 1 and beta 1 the updated state maps k to v) and a
float64 step; fast_exp (Cephes' expf, kernels.hpp:142-163) within 2 ulp of exp; and the reference's invariants on
the states: a verify equals one token at a time, a tree row the chain of its ancestors, verify + keep the verify of
the kept prefix (the states taken back from the kept row's, model.cpp:1617-1633), bit for bit."""
import numpy as np
import pytest

import pyoracle as po
from f64_model import GDN_MISTAKES, F64Model, topk_margin
from model_helpers import rel_err, tree_parents

GDN = dict(hidden=128, vocab=256, n_layers=3, n_experts=8, top_k=2, moe_ff=64, shared_ff=64, n_heads=4, n_kv_heads=2,
           head_dim=32, rope_dim=16, rope_theta=1e4, eps=1e-6, max_ctx=96, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32,
           gdn_v_dim=32, conv_kernel=4, gdn_layers=[1, 1, 0])
CTX = 30
SIGMA_R = 1.0 / np.sqrt(GDN["hidden"])
TOL = {1: 4e-6, 0: 4e-5}


def _models(seed=13):
    om = po.Model(GDN, seed=seed, router_sigma=SIGMA_R, ctx=CTX)
    return om, F64Model(om)


@pytest.mark.parametrize("mode", [1, 0])
@pytest.mark.parametrize("tree", [False, True])
def test_gdn_verify_matches_float64(mode, tree):
    om, fm = _models()
    parents = tree_parents((2, 2)) if tree else None
    n = 7 if tree else 5
    toks = (np.arange(n) * 41 + 5) % GDN["vocab"]
    om.position = CTX
    ol, oids = om.verify(toks, parents, mode=mode, route=True)
    fl, fids, fp = fm.verify(toks, CTX, parents, mode=mode)
    assert topk_margin(fp, GDN["top_k"]).min() > 1e-4, "routing near-tie: pick another seed"
    assert np.array_equal(oids, fids)
    err = rel_err(ol, fl)
    assert err <= TOL[mode], f"logits differ from float64 by {err:.3e} (mode {mode})"


@pytest.mark.parametrize("mistake", GDN_MISTAKES)
def test_gdn_planted_mistakes_are_caught(mistake):
    om, fm = _models()
    toks = np.array([3, 77, 150, 201, 9], np.int32)
    om.position = CTX
    ol, oids = om.verify(toks, mode=1, route=True)
    fl, fids, _ = fm.verify(toks, CTX, None, mode=1, mistakes=(mistake,))
    err = rel_err(ol, fl)
    assert err > 5 * TOL[1] or not np.array_equal(oids, fids), f"{mistake}: only {err:.3e} away"


def test_delta_rule_defining_property():
    """decay 1, beta 1, |k| = 1: the updated state maps k to v exactly (S' = S + k (v - S^T k)^T, so S'^T k = v)"""
    rng = np.random.default_rng(1)
    dk, dv = 32, 48
    S = rng.standard_normal((dk, dv)).astype(np.float32) * 0.3
    k = rng.standard_normal(dk)
    k = (k / np.linalg.norm(k)).astype(np.float32)
    q, v = rng.standard_normal(dk).astype(np.float32), rng.standard_normal(dv).astype(np.float32)
    S1, out = po.gdn_step(S, q, k, v, 1.0, 1.0)
    np.testing.assert_allclose(S1.astype(np.float64).T @ k, v, atol=2e-5)
    np.testing.assert_allclose(out, S1.astype(np.float64).T @ q, rtol=1e-5, atol=1e-6)
    # general decay and beta against float64
    S64 = S.astype(np.float64) * 0.8
    delta = (v - S64.T @ k) * 0.3
    S64 += np.outer(k, delta)
    S2, out2 = po.gdn_step(S, q, k, v, 0.8, 0.3)
    np.testing.assert_allclose(S2, S64, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out2, S64.T @ q, rtol=1e-5, atol=1e-6)


def test_fast_exp_within_two_ulp():
    xs = np.concatenate([np.linspace(-87, 88, 20001), np.random.default_rng(2).uniform(-30, 30, 5000)])
    for x in xs.astype(np.float32):
        got = np.float32(po.fast_exp(float(x)))
        want = np.float32(np.exp(np.float64(x)))
        assert abs(int(got.view(np.int32)) - int(want.view(np.int32))) <= 2, (x, got, want)
    assert np.float32(po.fast_exp(-200.0)) == np.float32(po.fast_exp(-87.0))


def test_gdn_batch_equals_one_at_a_time():
    a, _ = _models()
    b, _ = _models()
    toks = np.array([11, 200, 37, 5, 99], np.int32)
    a.position = b.position = CTX
    batch = a.verify(toks)
    single = np.concatenate([b.verify(toks[i:i + 1]) for i in range(5)])
    assert np.array_equal(batch.view(np.uint32), single.view(np.uint32))


def test_gdn_tree_row_equals_its_ancestors_chain():
    par = tree_parents((2, 2))   # 7 rows
    toks = ((np.arange(7) * 29 + 3) % GDN["vocab"]).astype(np.int32)
    a, _ = _models()
    a.position = CTX
    tree = a.verify(toks, par)
    for row in (3, 4, 6):
        chain = [row]
        while par[chain[-1]] >= 0:
            chain.append(par[chain[-1]])
        chain = chain[::-1]
        b, _ = _models()
        b.position = CTX
        got = b.verify(toks[chain])[-1]
        assert np.array_equal(got.view(np.uint32), tree[row].view(np.uint32)), row


@pytest.mark.parametrize("tree", [False, True])
def test_gdn_keep_equals_verify_of_the_kept_prefix(tree):
    par = tree_parents((2, 2)) if tree else None
    n = 7 if tree else 5
    toks = ((np.arange(n) * 17 + 8) % GDN["vocab"]).astype(np.int32)
    path = np.array([0, 2, 6], np.int32) if tree else None   # a root-to-leaf path of the (2, 2) tree
    kept = 3
    nxt = np.array([42, 7], np.int32)
    a, _ = _models()
    a.position = CTX
    a.verify(toks, par)
    a.keep(kept, path)
    got = a.verify(nxt)
    b, _ = _models()
    b.position = CTX
    b.verify(toks[path] if tree else toks[:kept])
    want = b.verify(nxt)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
