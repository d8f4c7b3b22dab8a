"""The oracle's MTP draft (oracle/oracle_layers.cpp orc_model_mtp / _draft / _draft_next, a restatement of
engine/src/model.cpp:1286-1479 and :4965-5039) pinned on the CPU: the pass against the float64 restatement in
tests/f64_model.py (both arithmetic modes, one and several rows), five planted slips of the composition each caught;
the draft is the first maximum of the logits and its probability the softmax closed form; the draft head's logits
are the full head's at its ids; a chained draft goes on from the last pass's mtp.norm output; the hidden rows default
to the last verify's final-normed rows (after a tree keep: the kept path's); and the reference's batching invariant
(n rows at once = one row at a time, bit for bit)."""
import numpy as np
import pytest

import pyoracle as po
from f64_model import MTP_MISTAKES, F64Model, mtp_pass
from model_helpers import rel_err, tree_parents

MTP = dict(hidden=128, vocab=256, n_layers=2, n_experts=8, top_k=2, moe_ff=64, shared_ff=64, n_heads=4, n_kv_heads=2,
           head_dim=32, rope_dim=16, rope_theta=1e4, eps=1e-6, max_ctx=96, max_rows=17, mtp=1)
CTX = 30
SIGMA_R = 1.0 / np.sqrt(MTP["hidden"])
TOL = {1: 4e-6, 0: 4e-5}


def _model(seed=13, ctx=CTX):
    return po.Model(MTP, seed=seed, router_sigma=SIGMA_R, ctx=ctx)


def _inputs(n, seed=1):
    rng = np.random.default_rng(seed)
    return rng.integers(0, MTP["vocab"], n).astype(np.int32), rng.normal(0, 1, (n, MTP["hidden"])).astype(np.float32)


@pytest.mark.parametrize("mode", [1, 0])
@pytest.mark.parametrize("n", [1, 4])
def test_mtp_matches_float64(mode, n):
    om = _model()
    fm = F64Model(om)
    toks, hid = _inputs(n)
    got = om.mtp(toks, CTX, hid, mode)
    want = mtp_pass(fm, toks, CTX, hid, mode)
    assert rel_err(got, want) <= TOL[mode]


@pytest.mark.parametrize("mistake", MTP_MISTAKES)
def test_each_planted_slip_is_caught(mistake):
    om = _model()
    fm = F64Model(om)
    toks, hid = _inputs(3)
    got = om.mtp(toks, CTX, hid, 1)
    want = mtp_pass(fm, toks, CTX, hid, 1, mistakes=(mistake,))
    assert rel_err(got, want) > 100 * TOL[1], mistake


def test_draft_is_the_first_maximum_with_its_softmax_probability():
    om = _model()
    toks, hid = _inputs(2)
    d, p, lg = om.draft(toks, CTX, hid)
    assert d == int(np.argmax(lg))
    l64 = lg.astype(np.float64)
    assert p == pytest.approx(1.0 / np.exp(l64 - l64[d]).sum(), rel=1e-6)
    # ties: the first maximum (std::max_element)
    om2 = _model()
    om2.set_draft_vocab([7, 7, 3])
    d2, _, lg2 = om2.draft(toks, CTX, hid)
    assert lg2[0] == lg2[1]
    assert d2 == (7 if lg2[0] >= lg2[2] else 3)


def test_draft_head_is_the_full_heads_rows():
    ids = np.array([200, 3, 77, 150, 9, 255, 0, 31], np.int32)
    full, sub = _model(), _model()
    sub.set_draft_vocab(ids)
    toks, hid = _inputs(3)
    _, _, lf = full.draft(toks, CTX, hid)
    d, p, ls = sub.draft(toks, CTX, hid)
    assert np.array_equal(ls, lf[ids])
    assert d == ids[int(np.argmax(ls))]
    l64 = ls.astype(np.float64)
    assert p == pytest.approx(1.0 / np.exp(l64 - l64.max()).sum(), rel=1e-6)


@pytest.mark.parametrize("mode", [1, 0])
def test_chained_draft_goes_on_from_the_mtp_output(mode):
    om = _model()
    fm = F64Model(om)
    toks, hid = _inputs(2)
    d1, _, _ = om.draft(toks, CTX, hid, mode)
    d2, _, lg2 = om.draft_next(d1, CTX + 2, mode)
    mtp_pass(fm, toks, CTX, hid, mode)
    want = mtp_pass(fm, [d1], CTX + 2, fm.mtp_out[None], mode)
    assert rel_err(lg2, want) <= TOL[mode]
    assert d2 == int(np.argmax(lg2))


def test_hidden_defaults_to_the_last_verifys_rows():
    a, b = _model(), _model()
    toks = np.array([5, 9, 11, 2], np.int32)
    a.verify(toks)
    b.verify(toks)
    hid = b.hidden()
    assert hid.shape == (4, MTP["hidden"])
    nxt = np.array([9, 11, 2, 40], np.int32)
    assert a.draft(nxt, CTX, None)[:2] == b.draft(nxt, CTX, hid)[:2]


def test_hidden_after_a_tree_keep_is_the_paths_rows():
    par = tree_parents([4, 3, 1])
    a, b = _model(), _model()
    toks = np.arange(1, len(par) + 1, dtype=np.int32)
    a.verify(toks, par)
    b.verify(toks, par)
    path = [0, 2, 9]   # row 9: a child of row 2 (depth 2)
    assert par[9] == 2 and par[2] == 0
    a.keep(3, path)
    b.keep(3, path)
    hid = b.hidden()[path]
    nxt = np.array([3, 10, 44], np.int32)
    da, pa, la = a.draft(nxt, CTX, None)
    db, pb, lb = b.draft(nxt, CTX, hid)
    assert np.array_equal(la, lb) and (da, pa) == (db, pb)


@pytest.mark.parametrize("mode", [0, 1])
def test_rows_at_once_equal_one_at_a_time(mode):
    a, b = _model(), _model()
    toks, hid = _inputs(5)
    la = a.mtp(toks, CTX, hid, mode)
    for t in range(4):
        b.mtp(toks[t:t + 1], CTX + t, hid[t:t + 1], mode, logits=False)
    lb = b.mtp(toks[4:], CTX + 4, hid[4:], mode)
    assert np.array_equal(la, lb)


def test_mtp_layer_kv_is_its_own():
    """the MTP pass writes the MTP layer's KV at its positions and no main layer's"""
    om = _model()
    before = [om.tensor(po.KV, l)[0].copy() for l in range(MTP["n_layers"] + 1)]
    toks, hid = _inputs(2)
    om.mtp(toks, CTX, hid)
    after = [om.tensor(po.KV, l)[0] for l in range(MTP["n_layers"] + 1)]
    for l in range(MTP["n_layers"]):
        assert np.array_equal(before[l], after[l])
    kv_row = MTP["n_kv_heads"] * MTP["head_dim"]
    diff = (before[-1] != after[-1]).view(np.uint16).reshape(2, MTP["max_ctx"], kv_row).any(axis=(0, 2))
    assert set(np.nonzero(diff)[0]) == {CTX, CTX + 1}
