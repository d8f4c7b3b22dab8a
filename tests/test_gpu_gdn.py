"""GPU parity of the Gated DeltaNet verify (gdn.hip; engine/src/model.cpp:3497-3688) against the oracle on the same
seeded inputs: a model of two Gated DeltaNet layers and a gated-attention layer, at small heads and at the real
model's head shape (dk = dv = 128). Logits within 1e-2 (max error over max |logit|), routed experts identical, greedy
tokens identical away from near-ties, and the layers' states after the step (conv inputs and recurrent state) within
5e-3 of the oracle's; chain and draft tree; verify + keep (the states as after the last kept row, model.cpp:
1617-1633) followed by the next verify; a tree row equal to the chain of its ancestors; gv_model_layer leaving the
states as they were.

The int8 path's steps: the GPU sums the delta rule's products in another order than the oracle (each lane a quarter
of the rows, then the quarters) and its exp / log1p are not glibc's, a 1e-7 relative difference that can move an int8
activation code by a step further on (the output projection's operands: ~5e-4 of that row's mixer output, seen), so a
row's logits or a router logit by up to ~1e-2. Hence:
  - logits: within 1e-2 of the int8 CPU path, or, where that misses, the reference's own GPU criterion
    (engine/src/gpu_check.cpp:80-94): against the exact path (fp32 activations, the oracle's mode 1, from the same
    states) the GPU's largest error at most 1.5 x the int8 CPU path's + 1e-6 of the exact logits' scale;
  - routing: an expert swap is accepted only where the oracle's K-th and (K+1)-th router logits are within 0.01 (its
    own trace); the swapped row and every row after it are then left out of the logits check, and a layer's states
    out of the state check when a swap came before it.
Layer by layer from the same inputs the mixer agrees to ~3e-7 away from such a step (test_layer_by_layer)."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import adopt_oracle_model, near_tie_rows, rel_err, route_margins, tree_parents

pytestmark = pytest.mark.gpu

CTX = 100
BASE = dict(hidden=256, vocab=512, n_layers=3, n_experts=16, top_k=4, moe_ff=128, shared_ff=128, n_heads=4,
            n_kv_heads=2, head_dim=64, rope_dim=16, rope_theta=1e7, eps=1e-6, max_ctx=160, max_rows=17,
            gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4, gdn_layers=[1, 1, 0])
SHAPES = {"small": BASE, "wide": dict(BASE, gdn_k_dim=128, gdn_v_dim=128)}
GDN_LAYERS = (0, 1)
STATE_TOL = 5e-3
TIE = 0.01   # router logit gap under which an expert swap is a near-tie


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


class Pair:
    """the oracle model and the GPU model with the same tensors, and the layers' first states to go back to"""

    def __init__(self, gv, cfg):
        self.gv, self.cfg = gv, cfg
        self.om = po.Model(cfg, seed=11, router_sigma=1.0 / np.sqrt(cfg["hidden"]), ctx=CTX)
        self.gm = gv.VerifyModel(cfg)
        adopt_oracle_model(self.gm, self.om, CTX)
        self.first = {l: (self.om.tensor(po.GDN_CONV_ST, l)[0].copy(), self.om.tensor(po.GDN_S, l)[0].copy())
                      for l in GDN_LAYERS}

    def reset(self):
        for l, (cs, s) in self.first.items():
            self.om.tensor(po.GDN_CONV_ST, l)[0][:] = cs
            self.om.tensor(po.GDN_S, l)[0][:] = s
            self.gm.adopt(self.gv.GDN_CONV_ST, cs, layer=l)
            self.gm.adopt(self.gv.GDN_S, s, layer=l)
        self.om.position = CTX
        self.gm.position = CTX

    def check_states(self, step=(99, None)):
        """the GDN layers' states against the oracle's: within STATE_TOL, or (given the exact path's states of the
        step) no further from those than the oracle's int8 path is (gpu_check.cpp:93); layers after an expert swap
        are skipped"""
        swapped_before, exact = step
        for l in GDN_LAYERS:
            if l > swapped_before:
                continue
            conv, S = self.gm.gdn_state(l)
            oc = self.om.tensor(po.GDN_CONV_ST, l)[0].view(np.float32).reshape(conv.shape)
            os_ = self.om.tensor(po.GDN_S, l)[0].view(np.float32).reshape(S.shape)
            for what, g, c, e in (("conv", conv, oc, exact and exact[l][0]), ("recurrent", S, os_, exact and exact[l][1])):
                err = rel_err(g, c)
                if err <= STATE_TOL:
                    continue
                assert e is not None, f"layer {l} {what} state: {err:.3e}"
                e = e.view(np.float32).reshape(g.shape)
                e_gpu, e_cpu = np.abs(g - e).max(), np.abs(c - e).max()
                assert e_gpu <= 1.5 * e_cpu + 1e-6 * np.abs(e).max(), \
                    f"layer {l} {what} state: {err:.3e}; against the exact path GPU {e_gpu:.3e}, int8 CPU {e_cpu:.3e}"


@pytest.fixture(scope="module", params=sorted(SHAPES))
def pair(gv, request):
    p = Pair(gv, SHAPES[request.param])
    yield p
    p.gm.close()


def _verify(pair, toks, parents=None):
    """both models' verify; checks the step and returns the first layer with an expert swap (99: none)"""
    om = pair.om
    pos, snap = om.position, {l: (om.tensor(po.GDN_CONV_ST, l)[0].copy(), om.tensor(po.GDN_S, l)[0].copy())
                              for l in GDN_LAYERS}
    exact = om.verify(toks, parents, mode=1)   # the exact path from the same states, then back to them
    exact_states = {l: (om.tensor(po.GDN_CONV_ST, l)[0].copy(), om.tensor(po.GDN_S, l)[0].copy()) for l in GDN_LAYERS}
    for l, (cs, st) in snap.items():
        om.tensor(po.GDN_CONV_ST, l)[0][:] = cs
        om.tensor(po.GDN_S, l)[0][:] = st
    om.position = pos
    ol, oids, tr = om.verify_trace(toks, parents)   # (its KV rows overwrite the exact path's)
    gl = pair.gm.verify(toks, parents=parents)
    gids = pair.gm.route_ids(len(toks))
    margins = route_margins(pair.om, tr)
    swaps = np.argwhere((oids != gids).any(axis=2))
    for l, r in swaps:
        assert margins[l, r] < TIE, f"experts differ at layer {l} row {r} (router gap {margins[l, r]:.3e})"
    first_row = int(swaps[:, 1].min()) if len(swaps) else len(toks)
    keep = slice(0, first_row)   # (rows in BFS order: a swapped row's descendants come after it)
    if first_row > 0:
        err = rel_err(gl[keep], ol[keep])
        if err > 1e-2:   # gpu_check.cpp:93
            e_gpu, e_cpu = np.abs(gl[keep] - exact[keep]).max(), np.abs(ol[keep] - exact[keep]).max()
            ref = np.abs(exact[keep]).max()
            assert e_gpu <= 1.5 * e_cpu + 1e-6 * ref, \
                f"logits max error {err:.3e}; against the exact path GPU {e_gpu / ref:.3e}, int8 CPU {e_cpu / ref:.3e}"
        ties = near_tie_rows(ol[keep], 2 * np.abs(gl[keep] - ol[keep]).max())
        for r in range(first_row):
            if r not in ties:
                assert np.argmax(gl[r]) == np.argmax(ol[r]), f"greedy token differs at row {r}"
    return (int(swaps[:, 0].min()) if len(swaps) else 99), exact_states


def _tokens(n, a=37, b=11):
    return (np.arange(n) * a + b) % BASE["vocab"]


@pytest.mark.parametrize("n", [1, 2, 5, 17])
def test_chain_verify(pair, n):
    pair.reset()
    pair.check_states(_verify(pair, _tokens(n)))


def test_tree_verify(pair):
    pair.reset()
    parents = tree_parents((4, 3))
    toks = _tokens(parents.size, 53, 5)
    pair.check_states(_verify(pair, toks, parents))   # (no keep: the states as after the last row)


def test_chain_keep_then_verify(pair):
    pair.reset()
    first, _ = _verify(pair, _tokens(5))
    pair.om.keep(3)
    pair.gm.keep(3)
    pair.check_states((first, None))
    second, exact = _verify(pair, _tokens(4, 29, 3))
    pair.check_states((min(first, second), exact))


def test_tree_keep_then_verify(pair):
    pair.reset()
    parents = tree_parents((4, 3))
    toks = _tokens(parents.size, 53, 5)
    first, _ = _verify(pair, toks, parents)
    path = [0, 2, 9]
    assert parents[2] == 0 and parents[9] == 2
    pair.om.keep(3, path)
    pair.gm.keep(3, path)
    pair.check_states((first, None))
    second, exact = _verify(pair, _tokens(5, 31, 7))
    pair.check_states((min(first, second), exact))


@pytest.mark.parametrize("tree", [False, True])
def test_layer_by_layer(pair, tree):
    """each layer fed the oracle's own input for it (gv_model_layer on the oracle's trace, from the same states): the
    residual after the mixer and after the MoE within 1e-5, the routed experts identical"""
    parents = tree_parents((4, 3)) if tree else None
    toks = _tokens(17, 53, 5)
    pair.reset()
    _, oids, tr = pair.om.verify_trace(toks, parents)
    for l in range(pair.cfg["n_layers"]):
        mid, out, ids = pair.gm.layer(l, tr[l, 0], parents)
        assert rel_err(mid, tr[l, 1]) <= 1e-5, f"layer {l} after the mixer: {rel_err(mid, tr[l, 1]):.3e}"
        assert np.array_equal(ids, oids[l]), f"layer {l} routing"
        want = tr[l, 1] + tr[l, 3]
        assert rel_err(out, want) <= 1e-5, f"layer {l} after the MoE: {rel_err(out, want):.3e}"


def test_tree_row_equals_chain_of_its_ancestors(pair):
    """on the GPU alone: a tree row's logits equal those of the chain through its ancestors from the same states"""
    parents = tree_parents((4, 3))
    toks = _tokens(parents.size, 53, 5)
    pair.reset()
    tl = pair.gm.verify(toks, parents=parents)
    for node in (1, 4, 5, 16):
        path = [node]
        while parents[path[-1]] >= 0:
            path.append(int(parents[path[-1]]))
        path = path[::-1]
        pair.reset()
        cl = pair.gm.verify(toks[path])
        assert rel_err(tl[node], cl[-1]) <= 1e-5, f"node {node}"


def test_one_token_at_a_time_equals_the_chain(pair):
    """verify of 5 rows = 5 verifies of one row each (the states carried from step to step)"""
    toks = _tokens(5, 41, 9)
    pair.reset()
    whole = pair.gm.verify(toks)
    pair.reset()
    ones = np.concatenate([pair.gm.verify(toks[i:i + 1]) for i in range(5)])
    assert rel_err(ones, whole) <= 1e-5


@pytest.mark.parametrize("tree", [False, True])
def test_fused_launch_equals_the_phases_apart(pair, tree):
    """the Gated DeltaNet layer's one launch (the a / b dots as its first workgroups) against the a / b dots in a
    launch of their own (gv_model_set_fused(0)): the same logits and states, bit for bit"""
    parents = tree_parents((4, 3)) if tree else None
    toks = _tokens(17 if tree else 5, 43, 2)
    pair.reset()
    fused = pair.gm.verify(toks, parents=parents)
    fs = [pair.gm.gdn_state(l) for l in GDN_LAYERS]
    pair.gm.set_fused(False)
    try:
        pair.reset()
        apart = pair.gm.verify(toks, parents=parents)
        ps = [pair.gm.gdn_state(l) for l in GDN_LAYERS]
    finally:
        pair.gm.set_fused(True)
    assert np.array_equal(fused, apart)
    for (c0, s0), (c1, s1) in zip(fs, ps):
        assert np.array_equal(c0, c1) and np.array_equal(s0, s1)


def test_layer_call_leaves_the_states(pair):
    pair.reset()
    before = [pair.gm.gdn_state(l) for l in GDN_LAYERS]
    x = np.random.default_rng(2).standard_normal((5, BASE["hidden"])).astype(np.float32)
    pair.gm.layer(0, x)
    for l, (c0, s0) in zip(GDN_LAYERS, before):
        c1, s1 = pair.gm.gdn_state(l)
        assert np.array_equal(c0, c1) and np.array_equal(s0, s1)


def test_randomized_gdn_model_runs(gv):
    gm = gv.VerifyModel(SHAPES["wide"])
    gm.randomize(5, ctx=CTX)
    tl = gm.verify(_tokens(17), parents=tree_parents((4, 3)))
    assert np.isfinite(tl).all() and np.abs(tl).max() > 0
    conv, S = gm.gdn_state(0)
    assert np.isfinite(S).all() and np.abs(S).max() > 0
    gm.close()
