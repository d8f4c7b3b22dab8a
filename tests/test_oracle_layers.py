"""The CPU oracle's layer functions (oracle/oracle_layers.cpp: attention, the MoE block, the whole verify step) pinned
against an independent float64 restatement written from the reference's formulas (tests/f64_model.py), on small
seeded models, in both arithmetic modes; plus the reference's own invariants (the attention's bits do not depend on
its block size beyond the merge, model.cpp:3799-3855). Each plausible slip in the composition (a dropped 1/sqrt(hd),
a RoPE sign or pairing, a missing gate, the q/k norm's (1 + w), the routed weights' renormalisation, silu, the mask,
the fp16 KV rounding) is planted in the restatement and must move it far outside the tolerance, so the comparison
is shown to catch it."""
import numpy as np
import pytest

import pyoracle as po
from f64_model import MISTAKES, F64Model, topk_margin
from model_helpers import rel_err, tree_parents

TINY = dict(hidden=128, vocab=256, n_layers=2, n_experts=8, top_k=2, moe_ff=64, shared_ff=64, n_heads=4, n_kv_heads=2,
            head_dim=32, rope_dim=16, rope_theta=1e4, eps=1e-6, max_ctx=96)
CTX = 40
SIGMA_R = 1.0 / np.sqrt(TINY["hidden"])
# oracle (fp32 sums) against float64: the exact path agrees to fp32 rounding amplified through two layers; the int8
# path re-quantizes every product's input, where an fp32 and a float64 value can round to neighbouring codes
TOL = {1: 4e-6, 0: 4e-5}


def _models(seed, attn_block=1024, cfg=TINY):
    om = po.Model(dict(cfg, attn_block=attn_block), seed=seed, router_sigma=SIGMA_R, ctx=CTX)
    return om, F64Model(om)


@pytest.fixture(scope="module")
def pair():
    return _models(11)


def _verify_both(om, fm, toks, parents, mode, mistakes=()):
    om.position = CTX
    ol, oids = om.verify(toks, parents, mode=mode, route=True)
    fl, fids, fp = fm.verify(toks, CTX, parents, mode=mode, mistakes=mistakes)
    return ol, oids, fl, fids, fp


@pytest.mark.parametrize("mode", [1, 0])
@pytest.mark.parametrize("tree", [False, True])
def test_verify_matches_float64(pair, mode, tree):
    om, fm = pair
    parents = tree_parents((2, 2)) if tree else None
    n = 7 if tree else 5
    toks = (np.arange(n) * 53 + 7) % TINY["vocab"]
    ol, oids, fl, fids, fp = _verify_both(om, fm, toks, parents, mode)
    margin = topk_margin(fp, TINY["top_k"]).min()
    assert margin > 1e-4, f"routing near-tie in the float64 model (margin {margin:.2e}): pick another seed"
    assert np.array_equal(oids, fids), "routed experts differ from the float64 restatement"
    err = rel_err(ol, fl)
    assert err <= TOL[mode], f"logits differ from float64 by {err:.3e} (mode {mode})"


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistakes_are_caught(pair, mistake):
    """each slip moves the restatement at least 5x the tolerance away from the oracle (or changes the routing)"""
    om, fm = pair
    toks = np.array([3, 77, 150, 201, 9], np.int32)
    ol, oids, fl, fids, _ = _verify_both(om, fm, toks, None, 1, mistakes=(mistake,))
    err = rel_err(ol, fl)
    assert err > 5 * TOL[1] or not np.array_equal(oids, fids), f"{mistake}: only {err:.3e} away"


def test_attention_block_size_invariance():
    """attend's blocks (GEODE_ATTN_BLOCK, model.cpp:344, :3799-3855): the bits of each block merge are fp32 rounding
    of the same softmax, so 1024-, 64- and 16-position blocks agree to fp32 rounding"""
    toks = np.array([5, 99, 180, 33, 240], np.int32)
    outs = []
    for blk in (1024, 64, 16):
        om = po.Model(dict(TINY, attn_block=blk), seed=11, router_sigma=SIGMA_R, ctx=CTX)
        outs.append(om.verify(toks, mode=1))
    assert rel_err(outs[1], outs[0]) <= 2e-6
    assert rel_err(outs[2], outs[0]) <= 2e-6


@pytest.mark.parametrize("mode", [1, 0])
def test_moe_layer_against_dense_brute_force(pair, mode):
    """orc_moe_layer (model.cpp:4123-4587) against every expert computed densely in float64 and weighted by the
    renormalised top-K probabilities (unpicked experts weighted 0), given router logits and the layer's own router"""
    om, fm = pair
    c = TINY
    M, H, E, K, F = 5, c["hidden"], c["n_experts"], c["top_k"], c["moe_ff"]
    rng = np.random.default_rng(4)
    h = rng.standard_normal((M, H)).astype(np.float32)
    L = fm.layers[1]
    for given in (True, False):
        lg = rng.standard_normal((M, E)).astype(np.float32) if given else None
        got, gids, gw = po.moe_layer(om, 1, h, lg, mode=mode)
        h64 = h.astype(np.float64)
        lg64 = lg.astype(np.float64) if given else h64 @ L["router"].T
        p = np.exp(lg64 - lg64.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert topk_margin(p, K).min() > 1e-5
        dense_w = np.zeros((M, E))
        for t in range(M):
            top = np.lexsort((np.arange(E), -p[t]))[:K]
            dense_w[t, top] = p[t, top] / p[t, top].sum()
            assert list(gids[t]) == list(top)
            assert np.abs(gw[t] - dense_w[t, top]).max() <= 1e-6
        quant = (lambda x: fm._mm(np.eye(x.shape[-1]), x, 0)) if mode == 0 else (lambda x: x)
        sig = lambda x: 1.0 / (1.0 + np.exp(-x))
        want = np.zeros((M, H))
        for e in range(E):   # every expert, dense
            gu = quant(h64) @ L["gu"][e].T
            y = quant(gu[:, :F] * sig(gu[:, :F]) * gu[:, F:]) @ L["dn"][e].T
            want += dense_w[:, e:e + 1] * y
        g = quant(h64) @ L["sg"].T
        u = quant(h64) @ L["su"].T
        sh = quant(g * sig(g) * u) @ L["sd"].T
        want += sig(h64 @ L["sgate"])[:, None] * sh
        err = rel_err(got, want)
        assert err <= TOL[mode], f"MoE block differs from the dense float64 form by {err:.3e}"


def test_routing_ties_go_to_the_lower_index():
    """route_topk with exactly tied probabilities: the lower expert index ranks first (gpu8_kernels.inc:974-978)"""
    E, K = 16, 4
    lg = np.zeros(E, np.float32)
    lg[[3, 7, 9, 12]] = 2.0   # four equal maxima
    lg[[1, 5]] = 1.0
    ids, w = po.route_topk(lg, K)
    assert list(ids) == [3, 7, 9, 12]
    assert np.allclose(w, 0.25, atol=1e-7)
    ids, _ = po.route_topk(lg, 6)
    assert list(ids) == [3, 7, 9, 12, 1, 5]
