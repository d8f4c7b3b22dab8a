"""The acceptance rules' two sampling paths on the GPU against the oracle (po.accept_textbook, po.accept_match): the
candidate path (each row's nucleus decided among the elements above one logit: a top_p < 1 prefix of the full
vocabulary, or the top_k / cap candidates) and the full walks it hands a call to when a row is not decided there.
Each case checks the emitted tokens exactly and which path served the call (gv_sampler_paths).

Textbook rule: C2's trial shape; small, ragged and one-chunk vocabularies; k = 1 and k = 31 (63 rows); a tiny top_p
(one kept token); a peaked and a flat temperature; coarse logits (ties inside the collected bins); a rejection with
no residual mass (draft = target, u_acc = 1: the target row's own draw); rows whose nucleus spans most of the
vocabulary and top_p = 1 (the walks). Sample-and-match: C2's rows at the reference's cap of 1024, top_k 1, 50 and
3000 (top_p 1), ties at the cut, a peaked temperature with a presence penalty (the walks, the penalty applied once),
a cap above the candidate path's 4096 (the walks), stop lists of 3 and 40 tokens."""
import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def _trial(seed, k, V, sigma=3.0, noise=0.5, grid=None):
    target = po.normal(seed, (k + 1) * V, sigma).reshape(k + 1, V)
    draft = target[:k] + po.normal(seed + 1, k * V, noise).reshape(k, V)
    if grid:
        target = (np.round(target / grid) * grid).astype(np.float32)
        draft = (np.round(draft / grid) * grid).astype(np.float32)
    rng = np.random.default_rng(seed + 2)
    return target, draft, rng.random(k).astype(np.float32), rng.random(k).astype(np.float32), np.float32(rng.random())


def _run(gv, target, draft, T, top_p, ud, ua, ur):
    c0, w0 = gv.sampler_paths()
    got = gv.accept_textbook(target, draft, T, top_p, False, ud, ua, ur)
    c1, w1 = gv.sampler_paths()
    want = po.accept_textbook(target, draft, T, top_p, False, ud, ua, ur)
    assert list(got) == list(want), (list(got), list(want))
    assert (c1 - c0) + (w1 - w0) == 1
    return "candidate" if c1 > c0 else "walks"


def _rejections(gv, target, draft, T, top_p, ud, ur):
    """every draft position rejected in turn (the residual draw), then all accepted (the bonus)"""
    k = draft.shape[0]
    paths = set()
    for first in range(min(k, 4) + 1):
        ua = np.zeros(k, np.float32)
        if first < k:
            ua[first] = np.float32(0.999999)
        paths.add(_run(gv, target, draft, T, top_p, ud, ua, ur))
    return paths


@pytest.mark.parametrize("seed", [5, 6, 7])
def test_c2_shape_takes_the_candidate_path(gv, seed):
    target, draft, ud, ua, ur = _trial(seed * 10, 4, 151936)
    assert _run(gv, target, draft, 0.7, 0.95, ud, ua, ur) == "candidate"
    assert _rejections(gv, target, draft, 0.7, 0.95, ud, ur) == {"candidate"}


@pytest.mark.parametrize("V", [1000, 4096, 4097, 12289, 50000])
def test_small_and_ragged_vocabularies(gv, V):
    target, draft, ud, _, ur = _trial(300 + V, 4, V)
    assert _rejections(gv, target, draft, 0.7, 0.95, ud, ur) == {"candidate"}


@pytest.mark.parametrize("k", [1, 31])
def test_chain_lengths(gv, k):
    target, draft, ud, ua, ur = _trial(400 + k, k, 20000)
    assert _run(gv, target, draft, 0.7, 0.95, ud, ua, ur) == "candidate"
    ua[:] = 0.0   # every draft stands: the bonus from row k
    assert _run(gv, target, draft, 0.7, 0.95, ud, ua, ur) == "candidate"


def test_tiny_top_p(gv):
    target, draft, ud, _, ur = _trial(500, 4, 151936)
    assert _rejections(gv, target, draft, 0.7, 1e-4, ud, ur) == {"candidate"}


@pytest.mark.parametrize("T", [0.05, 2.0])
def test_temperatures(gv, T):
    target, draft, ud, _, ur = _trial(600, 4, 151936)
    _rejections(gv, target, draft, T, 0.95, ud, ur)   # (either path; the tokens must match)


def test_ties_inside_the_collected_bins(gv):
    """logits on a 1/8 grid: equal values straddle the top-p prefix's end and the draws, taken in index order"""
    target, draft, ud, _, ur = _trial(700, 4, 151936, grid=0.125)
    assert _rejections(gv, target, draft, 0.7, 0.95, ud, ur) == {"candidate"}


def test_rejection_without_residual_mass(gv):
    """draft = target and u_acc = 1: q(d) = p(d) and the first draft is rejected with max(0, p - q) = 0 everywhere,
    so the emitted token is the target row's own draw"""
    target, _, ud, _, ur = _trial(800, 4, 151936)
    draft = target[:4].copy()
    ua = np.ones(4, np.float32)
    assert _run(gv, target, draft, 0.7, 0.95, ud, ua, ur) == "candidate"


def test_flat_rows_and_top_p_one_take_the_walks(gv):
    target, draft, ud, _, ur = _trial(900, 4, 151936, sigma=1.0)   # T = 1 on N(0, 1): most of the vocabulary
    assert _rejections(gv, target, draft, 1.0, 0.95, ud, ur) == {"walks"}
    target, draft, ud, _, ur = _trial(901, 4, 151936)
    assert _rejections(gv, target, draft, 0.7, 1.0, ud, ur) == {"walks"}


# ---------------------------------------------------------------- sample-and-match (the top_k / cap candidates)
def _match(gv, logits, batch, T, top_p, top_k, cap, u):
    c0, w0 = gv.sampler_paths()
    got = gv.accept_match(logits, batch, T, top_p, top_k, cap, u)
    c1, w1 = gv.sampler_paths()
    want = po.accept_match(logits, batch, T, top_p, top_k, cap, u)
    assert list(got[0]) == list(want[0]) and got[1] == want[1], (got, want)
    assert (c1 - c0) + (w1 - w0) == 1
    return "candidate" if c1 > c0 else "walks"


def _match_case(seed, V=151936, n=5, sigma=3.0):
    x = po.normal(seed, n * V, sigma).reshape(n, V)
    rng = np.random.default_rng(seed + 1)
    u = rng.random(n)
    # drafts: what each row samples on some trials (so that they stand), another token on others
    return x, u, rng


@pytest.mark.parametrize("seed", [11, 12])
def test_match_c2_shape_takes_the_candidate_path(gv, seed):
    x, u, rng = _match_case(seed * 10)
    for trial in range(4):
        samples = [po.sample(x[i], 0.7, 0.95, 0, 1024, u[i]) for i in range(5)]
        batch = np.array([7] + samples[:4], np.int32)
        if trial % 2:
            batch[1 + trial % 4] = (batch[1 + trial % 4] + 1) % x.shape[1]
        assert _match(gv, x, batch, 0.7, 0.95, 0, 1024, u) == "candidate"
        u = rng.random(5)


@pytest.mark.parametrize("top_k,top_p", [(50, 0.9), (1, 0.95), (3000, 1.0)])
def test_match_top_k(gv, top_k, top_p):
    x, u, _ = _match_case(1300 + top_k)
    samples = [po.sample(x[i], 0.7, top_p, top_k, 1024, u[i]) for i in range(5)]
    batch = np.array([7] + samples[:4], np.int32)
    assert _match(gv, x, batch, 0.7, top_p, top_k, 1024, u) == "candidate"


def test_match_ties_in_the_cut_bin(gv):
    """logits on a 1/4 grid: the 1024th candidate sits among many equal values, taken in index order"""
    x, u, _ = _match_case(1400)
    x = (np.round(x * 4.0) / 4.0).astype(np.float32)
    samples = [po.sample(x[i], 0.7, 0.95, 0, 1024, u[i]) for i in range(5)]
    batch = np.array([7] + samples[:4], np.int32)
    _match(gv, x, batch, 0.7, 0.95, 0, 1024, u)   # (either path: the tokens must match)


def test_match_walks_with_penalty_applied_once(gv):
    """T = 0.05: the top 1024 reach below the candidate path's bins, so the call goes to the walks after the presence
    penalty was applied in place: the penalized logits and tokens must match the oracle's (no second penalty)"""
    V = 151936
    x = po.normal(1500, 5 * V, 3.0).reshape(5, V)
    u = np.random.default_rng(1501).random(5)
    seen = np.random.default_rng(1502).choice(V, size=300, replace=False).astype(np.int32)
    batch = [11, 1, 2, 3, 4]
    c0, w0 = gv.sampler_paths()
    want, wk, wlg = po.accept_match_ex(x, batch, 0.05, 0.95, 0, 1024, u, seen, 1.5)
    got, gk, glg = gv.accept_match_ex(x, batch, 0.05, 0.95, 0, 1024, u, seen, 1.5)
    c1, w1 = gv.sampler_paths()
    assert (c1, w1) == (c0, w0 + 1)
    assert list(got) == list(want) and gk == wk
    for r in range(wk):
        assert np.array_equal(glg[r].view(np.uint32), wlg[r].view(np.uint32))


def test_match_large_cap_takes_the_walks(gv):
    x, u, _ = _match_case(1600)
    batch = np.array([7, 1, 2, 3, 4], np.int32)
    assert _match(gv, x, batch, 0.7, 0.95, 0, 8192, u) == "walks"


@pytest.mark.parametrize("n_stop", [3, 40])
def test_match_stop_lists_on_the_candidate_path(gv, n_stop):
    """stop tokens with no penalty: up to 32 go to the launch as kernel arguments (no copies), more through the copied
    inputs; a draft that is a stop token never stands, on both"""
    x, u, rng = _match_case(1700 + n_stop)
    samples = [po.sample(x[i], 0.7, 0.95, 0, 1024, u[i]) for i in range(5)]
    batch = np.array([7] + samples[:4], np.int32)
    stop = np.concatenate([[samples[1]], rng.choice(x.shape[1], size=n_stop - 1, replace=False)]).astype(np.int32)
    none = np.zeros(0, np.int32)
    c0, w0 = gv.sampler_paths()
    want, wk, _ = po.accept_match_ex(x, batch, 0.7, 0.95, 0, 1024, u, none, 0.0, stop)
    got, gk, _ = gv.accept_match_ex(x, batch, 0.7, 0.95, 0, 1024, u, none, 0.0, stop)
    c1, w1 = gv.sampler_paths()
    assert list(got) == list(want) and gk == wk, (list(got), list(want))
    assert (c1, w1) == (c0 + 1, w0)
    assert wk <= 2   # (row 1's sample is a stop token: its draft cannot stand)
