"""GPU parity of the sampler and the acceptance rules (C2) against the oracle, on C2's shapes: logits rows of
V = 151,936 ~ N(0, 3), T = 0.7, top-p 0.95, seeded uniforms. The sampled indices are compared exactly; the GPU's
double sums run in another order, which could move a pick only when a uniform falls within ~1e-15 of a boundary."""
import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu

V = 151936


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def _rows(seed, n, sigma=3.0, v=V):
    return po.normal(seed, n * v, sigma).reshape(n, v)


def _uniforms(seed, n):
    return np.random.default_rng(seed).random(n)


def test_greedy_is_the_first_argmax(gv):
    x = _rows(1, 5)
    x[3, 100] = x[3, 7] = x[3].max() + 1.0   # a tie for the maximum: the lower index wins
    got = gv.sample_rows(x, 0.0)
    want = [po.sample(x[r], 0.0, 1.0) for r in range(5)]
    assert list(got) == want
    assert got[3] == 7


@pytest.mark.parametrize("seed", [2, 3, 4])
def test_sampler_c2(gv, seed):
    """the reference's default: the top 1024 candidates, T = 0.7, top-p 0.95, one uniform a row"""
    x = _rows(seed, 5)
    for rep in range(4):
        u = _uniforms(100 * seed + rep, 5)
        got = gv.sample_rows(x, 0.7, 0.95, 0, 1024, u)
        want = [po.sample(x[r], 0.7, 0.95, 0, 1024, u[r]) for r in range(5)]
        assert list(got) == want, (rep, list(got), want)


def test_sampler_top_k(gv):
    x = _rows(5, 4)
    u = _uniforms(5, 4)
    got = gv.sample_rows(x, 1.0, 0.9, 40, 1024, u)
    assert list(got) == [po.sample(x[r], 1.0, 0.9, 40, 1024, u[r]) for r in range(4)]


def test_sampler_ties_at_the_threshold(gv):
    """logits on a coarse grid: hundreds of equal values around the 1024th; the lower indices are the candidates"""
    x = np.round(_rows(6, 3) * 2.0).astype(np.float32) / 2.0
    for rep in range(4):
        u = _uniforms(60 + rep, 3)
        got = gv.sample_rows(x, 1.5, 0.999, 0, 1024, u)
        assert list(got) == [po.sample(x[r], 1.5, 0.999, 0, 1024, u[r]) for r in range(3)]


def test_sampler_full_vocabulary_nucleus(gv):
    x = _rows(7, 3)
    u = _uniforms(7, 3)
    got = gv.sample_rows(x, 0.7, 0.95, 0, 0, u)
    assert list(got) == [po.sample(x[r], 0.7, 0.95, 0, 0, u[r]) for r in range(3)]


def test_small_vocabulary_every_candidate(gv):
    """V below the cap: every token is a candidate"""
    x = _rows(8, 4, 1.0, 300)
    for rep in range(3):
        u = _uniforms(80 + rep, 4)
        got = gv.sample_rows(x, 1.0, 1.0, 0, 1024, u)
        assert list(got) == [po.sample(x[r], 1.0, 1.0, 0, 1024, u[r]) for r in range(4)]


def test_sample_and_match(gv):
    """drafts that the rows sample stand; the first that is not ends the chain"""
    x = _rows(9, 5)
    u = _uniforms(9, 5)
    samples = [po.sample(x[r], 0.7, 0.95, 0, 1024, u[r]) for r in range(5)]
    for stood in range(5):   # the first `stood` drafts are what rows 0..stood-1 sample, the next one is not
        batch = [11] + [samples[i] for i in range(4)]
        if stood < 4:
            batch[stood + 1] = (samples[stood] + 1) % V
        got, kept = gv.accept_match(x, batch, 0.7, 0.95, 0, 1024, u)
        want, wkept = po.accept_match(x, batch, 0.7, 0.95, 0, 1024, u)
        assert list(got) == list(want) and kept == wkept
        assert kept == stood + 1


def _c2_trial(seed, k=4):
    target = _rows(seed, k + 1)
    draft = target[:k] + po.normal(seed + 1, k * V, 0.5).reshape(k, V)
    rng = np.random.default_rng(seed)
    return target, draft, rng.random(k).astype(np.float32), rng.random(k).astype(np.float32), np.float32(rng.random())


@pytest.mark.parametrize("seed", range(20, 32))
def test_textbook_rule_stochastic(gv, seed):
    target, draft, ud, ua, ur = _c2_trial(seed)
    got = gv.accept_textbook(target, draft, 0.7, 0.95, False, ud, ua, ur)
    want = po.accept_textbook(target, draft, 0.7, 0.95, False, ud, ua, ur)
    assert list(got) == list(want), (list(got), list(want))


def test_textbook_rule_rejections(gv):
    """acceptance uniforms near 1 force rejections at each position in turn (the residual draw)"""
    target, draft, ud, _, ur = _c2_trial(40)
    for first_reject in range(4):
        ua = np.zeros(4, np.float32)
        ua[first_reject] = np.float32(0.999999)
        got = gv.accept_textbook(target, draft, 0.7, 0.95, False, ud, ua, ur)
        want = po.accept_textbook(target, draft, 0.7, 0.95, False, ud, ua, ur)
        assert list(got) == list(want)


def test_textbook_rule_greedy(gv):
    target, draft, ud, ua, ur = _c2_trial(50)
    draft[:2] = target[:2]   # the first two drafts agree with the target's argmax
    got = gv.accept_textbook(target, draft, 0.7, 0.95, True, ud, ua, ur)
    want = po.accept_textbook(target, draft, 0.7, 0.95, True, ud, ua, ur)
    assert list(got) == list(want)
    assert len(got) >= 3


@pytest.mark.parametrize("temp", [0.0, 0.7])
def test_sample_and_match_presence_penalty_and_stops(gv, temp):
    """the generate loop's presence penalty (geode.cpp:236-255) and stop tokens (:333) against the oracle: the same
    emitted tokens, kept rows and penalized logits; drafts built so that penalties change the samples"""
    x = _rows(91, 5, 1.0)
    u = _uniforms(91, 5)
    rng = np.random.default_rng(92)
    for trial in range(12):
        seen = rng.choice(V, size=int(rng.integers(0, 400)), replace=False).astype(np.int32)
        pen = float(rng.choice([0.5, 1.5, 4.0]))
        # drafts: what the oracle's penalized rows sample (so that they stand), one of them replaced on odd trials
        _, _, lg0 = po.accept_match_ex(x, [1, 2, 3, 4, 5], temp, 0.95, 0, 1024, u, seen, pen)
        batch = [11]
        for i in range(4):   # the row i sample with row i's penalty set (seen + the drafts before)
            out_i, _, _ = po.accept_match_ex(x[i:i + 1], [0], temp, 0.95, 0, 1024, u[i:i + 1],
                                             np.unique(np.concatenate([seen, batch[1:]])).astype(np.int32), pen)
            batch.append(int(out_i[0]))
        if trial % 2:
            batch[1 + trial % 4] = (batch[1 + trial % 4] + 1) % V
        stop = [batch[3]] if trial % 3 == 0 else []
        want, wk, wlg = po.accept_match_ex(x, batch, temp, 0.95, 0, 1024, u, seen, pen, stop)
        got, gk, glg = gv.accept_match_ex(x, batch, temp, 0.95, 0, 1024, u, seen, pen, stop)
        assert list(got) == list(want) and gk == wk, (trial, list(got), list(want))
        for r in range(wk):   # the rows that were sampled carry the same penalized logits
            assert np.array_equal(glg[r].view(np.uint32), wlg[r].view(np.uint32))


@pytest.mark.parametrize("top_p", [0.95, 1.0])
def test_full_vocabulary_flat_rows(gv, top_p):
    """T = 1 on N(0, 1) logits: the 0.95 nucleus holds most of the 151,936 tokens (no candidate limit)"""
    x = _rows(71, 4, 1.0)
    for rep in range(4):
        u = _uniforms(710 + rep, 4)
        got = gv.sample_rows(x, 1.0, top_p, 0, 0, u)
        assert list(got) == [po.sample(x[r], 1.0, top_p, 0, 0, u[r]) for r in range(4)], rep


def test_full_vocabulary_ties(gv):
    """logits on a coarse grid: thousands of equal values at the top-p boundary and at the draws; ties are taken in
    index order by both walks"""
    x = np.round(_rows(72, 3, 1.0) * 4.0).astype(np.float32) / 4.0
    for rep in range(6):
        u = _uniforms(720 + rep, 3)
        got = gv.sample_rows(x, 0.8, 0.9, 0, 0, u)
        assert list(got) == [po.sample(x[r], 0.8, 0.9, 0, 0, u[r]) for r in range(3)], rep


def test_textbook_rule_flat_and_tied_rows(gv):
    """the textbook rule where the nuclei span most of the vocabulary and where logits tie, rejections forced at each
    position in turn (the residual over the full vocabulary)"""
    for flat, coarse in ((True, False), (False, True)):
        sig = 1.0 if flat else 3.0
        target = _rows(73, 5, sig)
        draft = target[:4] + po.normal(74, 4 * V, 0.5).reshape(4, V)
        if coarse:
            target = np.round(target * 2.0).astype(np.float32) / 2.0
            draft = np.round(draft * 2.0).astype(np.float32) / 2.0
        rng = np.random.default_rng(75)
        ud, ur = rng.random(4).astype(np.float32), np.float32(rng.random())
        for first_reject in range(5):
            ua = np.zeros(4, np.float32)
            if first_reject < 4:
                ua[first_reject] = np.float32(0.999999)
            got = gv.accept_textbook(target, draft, 1.0, 0.95, False, ud, ua, ur)
            want = po.accept_textbook(target, draft, 1.0, 0.95, False, ud, ua, ur)
            assert list(got) == list(want), (flat, coarse, first_reject, list(got), list(want))
