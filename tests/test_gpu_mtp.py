"""GPU parity of the MTP draft layer (mtp.hip; engine/src/model.cpp:1286-1479, :4965-5039) against the oracle on the
same seeded weights: a main model of gated-attention layers (and one with Gated DeltaNet layers) plus its MTP layer.

Checked: the hidden rows a verify leaves (the final-normed rows) against the oracle's; the MTP pass's logits (last row,
whole vocabulary or a draft head) within 1e-2 of the int8 CPU path (max error over max |logit|) or, where that misses,
the reference's GPU criterion against the exact path (engine/src/gpu_check.cpp:80-94: the GPU's largest error at most
1.5 x the int8 CPU path's + 1e-6 of the exact logits' scale); the draft token equal to the oracle's away from
near-ties; the pick kernels exactly: the draft is the first maximum of the GPU's own logits and the probability the
closed form 1 / sum exp(l - max) of them (float64, 1e-6); the draft head's logits equal to the full head's at its ids
bit for bit; the hidden rows' default (the last verify's, or the kept path's after a tree keep) equal to passing them;
chained drafts (draft_next) against the oracle's; the generate loop's chain rule (geode.cpp:310-317) against a host
restatement on the oracle; a prompt's pass in chunks of max_rows followed by a draft."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import adopt_oracle_model, near_tie_rows, rel_err, tree_parents

pytestmark = pytest.mark.gpu

CTX = 60
ATTN = dict(hidden=256, vocab=512, n_layers=2, n_experts=16, top_k=4, moe_ff=128, shared_ff=128, n_heads=4,
            n_kv_heads=2, head_dim=64, rope_dim=16, rope_theta=1e7, eps=1e-6, max_ctx=160, max_rows=17, mtp=1)
GDN = dict(ATTN, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
           gdn_layers=[1, 0, 1])
SHAPES = {"attn": ATTN, "gdn": GDN}


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


class Pair:
    def __init__(self, gv, cfg):
        self.cfg = cfg
        self.om = po.Model(cfg, seed=21, router_sigma=1.0 / np.sqrt(cfg["hidden"]), ctx=CTX)
        self.gm = gv.VerifyModel(cfg)
        adopt_oracle_model(self.gm, self.om, CTX)


@pytest.fixture(scope="module", params=sorted(SHAPES))
def pair(gv, request):
    p = Pair(gv, SHAPES[request.param])
    yield p
    p.gm.close()


def _inputs(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(0, ATTN["vocab"], n).astype(np.int32),
            rng.normal(0, 1, (n, ATTN["hidden"])).astype(np.float32))


def _check_logits(gl, ol, exact):
    err = rel_err(gl, ol)
    if err > 1e-2:   # gpu_check.cpp:93
        e_gpu, e_cpu = np.abs(gl - exact).max(), np.abs(ol - exact).max()
        assert e_gpu <= 1.5 * e_cpu + 1e-6 * np.abs(exact).max(), \
            f"logits {err:.3e}; against the exact path GPU {e_gpu:.3e}, int8 CPU {e_cpu:.3e}"
    return err


def _check_pick(gm, d, p):
    """the pick kernels on the GPU's own logits: the first maximum (through the draft ids) and its probability"""
    gl = gm.draft_logits()
    best = int(np.argmax(gl))
    ids = getattr(gm, "_ids", None)
    assert d == (int(ids[best]) if ids is not None else best)
    l64 = gl.astype(np.float64)
    assert p == pytest.approx(1.0 / np.exp(l64 - l64[best]).sum(), rel=1e-6)
    return gl


def _draft_both(pair, toks, pos, hidden):
    """the oracle's exact-path logits, then its int8 draft (its MTP KV as the int8 path leaves it), then the GPU's"""
    om, gm = pair.om, pair.gm
    _, _, exact = om.draft(toks, pos, hidden, mode=1)
    od, op, ol = om.draft(toks, pos, hidden)
    d, p = gm.draft(toks, pos, hidden)
    gl = _check_pick(gm, d, p)
    _check_logits(gl, ol, exact)
    if not near_tie_rows(ol[None], 2 * np.abs(gl - ol).max() + 1e-6):
        assert d == od
        assert p == pytest.approx(op, rel=1e-2)
    return d, od


def test_hidden_rows_after_verify(pair):
    om, gm = pair.om, pair.gm
    om.position = gm.position = CTX
    toks = np.array([3, 77, 140, 5], np.int32)
    ol = om.verify(toks)
    gl = gm.verify(toks)
    assert rel_err(gl, ol) <= 1e-2
    gh, oh = gm.hidden(), om.hidden()
    assert gh.shape == oh.shape == (4, ATTN["hidden"])
    assert rel_err(gh, oh) <= 1e-2


@pytest.mark.parametrize("n", [1, 3, 8, 17])
def test_draft_matches_oracle(pair, n):
    toks, hid = _inputs(n, seed=n)
    _draft_both(pair, toks, CTX + 5, hid)


def test_draft_from_the_verify_rows(pair):
    """hidden None: the last verify's final-normed rows, equal to passing them (bit for bit), and against the oracle
    fed its own rows"""
    om, gm = pair.om, pair.gm
    om.position = gm.position = CTX
    toks = np.array([9, 200, 31, 4, 66], np.int32)
    om.verify(toks)
    gm.verify(toks)
    om.keep(3)
    gm.keep(3)
    nxt = np.array([200, 31, 8], np.int32)
    d0, p0 = gm.draft(nxt, CTX, None)
    l0 = gm.draft_logits()
    d1, p1 = gm.draft(nxt, CTX, gm.hidden()[:3])
    assert (d0, p0) == (d1, p1) and np.array_equal(l0, gm.draft_logits())
    _, _, exact = om.draft(nxt, CTX, None, mode=1)
    _, _, ol = om.draft(nxt, CTX, None)
    _check_logits(l0, ol, exact)


def test_draft_after_a_tree_keep(pair):
    om, gm = pair.om, pair.gm
    om.position = gm.position = CTX
    par = tree_parents((4, 3))
    toks = (np.arange(len(par)) * 7 + 3).astype(np.int32) % ATTN["vocab"]
    om.verify(toks, par)
    gm.verify(toks, parents=par)
    path = [0, 2, 9]   # row 9: a child of row 2 (depth 2)
    assert par[9] == 2 and par[2] == 0
    om.keep(3, path)
    gm.keep(3, path)
    nxt = np.array([toks[2], toks[9], 17], np.int32)
    d0, _ = gm.draft(nxt, CTX, None)
    l0 = gm.draft_logits()
    gm.draft(nxt, CTX, gm.hidden()[path])
    assert np.array_equal(l0, gm.draft_logits())
    _, _, exact = om.draft(nxt, CTX, None, mode=1)
    _, _, ol = om.draft(nxt, CTX, None)
    _check_logits(l0, ol, exact)


def test_chained_drafts_match_oracle(pair):
    """three chained drafts: each step's logits against the oracle fed the same tokens (the GPU's drafts), the exact
    path's chain first, then the int8 path's over it (the MTP KV then as the int8 path leaves it)"""
    om, gm = pair.om, pair.gm
    toks, hid = _inputs(2, seed=40)
    pos = CTX + 10
    d, p = gm.draft(toks, pos, hid)
    gls, feed = [_check_pick(gm, d, p)], [d]
    for q in range(pos + 2, pos + 5):
        d, p = gm.draft_next(feed[-1], q)
        gls.append(_check_pick(gm, d, p))
        feed.append(d)
    exact = [om.draft(toks, pos, hid, mode=1)[2]]
    exact += [om.draft_next(feed[j], pos + 2 + j, mode=1)[2] for j in range(3)]
    ols = [om.draft(toks, pos, hid)[2]]
    ols += [om.draft_next(feed[j], pos + 2 + j)[2] for j in range(3)]
    for g, o, e in zip(gls, ols, exact):
        _check_logits(g, o, e)


def test_draft_head_rows(pair):
    gm = pair.gm
    toks, hid = _inputs(3, seed=5)
    gm.set_draft_vocab(None)
    gm.draft(toks, CTX + 20, hid)
    full = gm.draft_logits()
    ids = np.array([500, 3, 77, 150, 9, 255, 0, 31, 400, 401, 402, 17, 18, 19, 20, 21, 300], np.int32)
    gm.set_draft_vocab(ids)
    gm._ids = ids
    try:
        d, p = gm.draft(toks, CTX + 20, hid)
        sub = _check_pick(gm, d, p)
        assert np.array_equal(sub, full[ids])
    finally:
        gm.set_draft_vocab(None)
        gm._ids = None


@pytest.mark.parametrize("pmin", [0.0, 1.01, "between"])
def test_chain_rule(pair, pmin):
    """gv_model_draft_chain against the generate loop's rule restated on the oracle (geode.cpp:301-317): the first
    draft always, further ones while the last probability >= pmin, kmax - 1 at most"""
    om, gm = pair.om, pair.gm
    om.position = gm.position = CTX
    toks, hid = _inputs(2, seed=77)
    pos, kmax = CTX + 30, 5

    def oracle_chain(pm):
        d, p, _ = om.draft(toks, pos, hid)
        out, probs, q = [d], [p], pos + 2
        while len(out) + 1 < kmax and p >= pm:
            d, p, _ = om.draft_next(out[-1], q)
            if p < pm:
                break
            out.append(d)
            probs.append(p)
            q += 1
        return out, probs

    if pmin == "between":   # a threshold that stops the chain at its third draft
        _, probs = oracle_chain(0.0)
        pm = float(probs[2]) * 1.001 if len(probs) > 2 else 0.5
    else:
        pm = pmin
    want, wp = oracle_chain(pm)
    got, gp = gm.draft_chain(toks, pos, kmax, pm, hid)
    if list(got) != want:
        pytest.skip(f"a near-tie in the chain: {list(got)} vs {want} (probabilities {list(gp)} vs {wp})")
    assert np.allclose(gp, wp, rtol=1e-2)
    if pmin == 0.0:
        assert len(got) == kmax - 1
    if pmin == 1.01:
        assert len(got) == 1


def test_prompt_pass_then_draft(pair):
    """gv_model_mtp_fill over 40 rows (three chunks of max_rows) then a draft that attends to them"""
    om, gm = pair.om, pair.gm
    toks, hid = _inputs(40, seed=9)
    om.mtp(toks, 10, hid, logits=False)
    gm.mtp_fill(toks, 10, hid)
    t2, h2 = _inputs(2, seed=10)
    _draft_both(pair, t2, 50, h2)


def test_refusals(gv, pair):
    gm = pair.gm
    toks, hid = _inputs(2, seed=1)
    with pytest.raises(gv.GeodeError):
        gm.draft(toks, ATTN["max_ctx"] - 1, hid)   # past the context
    with pytest.raises(gv.GeodeError):
        gm.draft(np.array([ATTN["vocab"]], np.int32), 0, hid[:1])
    with pytest.raises(gv.GeodeError):
        gm.set_draft_vocab([ATTN["vocab"]])


def test_graph_replays_match_direct_launches(gv, pair):
    """the MTP passes replayed from their graphs (captured on the second use of a row count) against direct launches:
    four rounds of a draft and two chained drafts at moving positions, bit for bit, the draft head switched after the
    second round (its graphs captured again)"""
    gm = pair.gm
    res = {}
    for graphs in (True, False):
        gm.set_graphs(graphs)
        out = []
        for r in range(4):
            if r in (0, 2):
                gm.set_draft_vocab(None if r == 0 else np.arange(3, 300, 2, dtype=np.int32))
            toks, hid = _inputs(3, seed=100 + r)
            pos = CTX + 4 * r
            out.append((gm.draft(toks, pos, hid), gm.draft_logits().copy()))
            d = out[-1][0][0]
            for q in range(2):
                out.append((gm.draft_next(d, pos + 3 + q), gm.draft_logits().copy()))
                d = out[-1][0][0]
        res[graphs] = out
    gm.set_graphs(True)
    gm.set_draft_vocab(None)
    for (a, la), (b, lb) in zip(res[True], res[False]):
        assert a == b and np.array_equal(la, lb)
