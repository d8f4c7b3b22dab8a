"""The sampler and the acceptance rules of the oracle pinned (CPU): the reference Sampler's own mt19937_64 draws
(golden fixture from oracle/_ref), a float64 restatement with injected uniforms, the top-p prefix property,
sample-and-match by brute force, and the textbook rule's output distribution equal to p (Leviathan et al. 2023,
Theorem 1) by integration over a grid of uniforms on a tiny vocabulary."""
import os

import numpy as np
import pytest

import pyoracle as po

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
P = po._ptr


def test_seeded_sampler_matches_reference_stream():
    lg = GOLDEN["sample_logits"]
    for (t, p, k, s), want in zip(GOLDEN["sample_settings"], GOLDEN["sample_draws"]):
        out = np.empty(64, np.int32)
        po.lib.orc_sample_seeded(P(lg), lg.size, float(t), float(p), int(k), int(s), 64, P(out))
        assert np.array_equal(out, want), (t, p, k, s)


def _nucleus64(lg, T, top_p, top_k=0, cap=1024):
    n = lg.size
    k = min(n, top_k if top_k > 0 else (cap if cap > 0 else n))
    order = sorted(range(n), key=lambda i: (-lg[i], i))[:k]
    mx = lg[order[0]]
    e = np.array([np.float32(np.exp(np.float32((lg[i] - mx) / np.float32(T)))) for i in order], np.float32)
    s = 0.0
    for v in e:
        s += float(v)
    keep = k
    if top_p < 1:
        acc = 0.0
        for i, v in enumerate(e):
            acc += float(v) / s
            if acc >= top_p:
                keep = i + 1
                break
    kept = sum(float(v) for v in e[:keep])
    return order, e, keep, kept


@pytest.mark.parametrize("T,top_p,top_k,cap", [(0.7, 0.95, 0, 1024), (1.0, 0.8, 20, 1024), (0.7, 0.95, 0, 0),
                                               (2.0, 1.0, 0, 64)])
def test_injected_uniform_sampler(T, top_p, top_k, cap):
    lg = po.normal(31, 2000, 3.0)
    for u in np.linspace(0.0, 0.999, 57):
        order, e, keep, kept = _nucleus64(lg, T, top_p, top_k, cap)
        r = kept * u
        want = order[keep - 1]
        for i in range(keep):
            r -= float(e[i])
            if r <= 0:
                want = order[i]
                break
        assert po.sample(lg, T, top_p, top_k, cap, float(u)) == want


def test_top_p_prefix_property_and_greedy():
    lg = po.normal(32, 500, 2.0)
    probs = po.nucleus_probs(lg, 0.7, 0.9)
    kept = np.flatnonzero(probs > 0)
    order = sorted(range(500), key=lambda i: (-lg[i], i))
    assert set(kept) == set(order[:kept.size])           # a prefix of the descending order
    full = np.exp(((lg - lg.max()) / np.float32(0.7)).astype(np.float32)).astype(np.float64)
    full /= full.sum()
    c = np.cumsum(full[order])
    assert c[kept.size - 1] >= 0.9 - 1e-12 and (kept.size == 1 or c[kept.size - 2] < 0.9)
    assert abs(probs.sum() - 1) < 1e-12
    lg2 = lg.copy()
    lg2[[10, 20]] = lg.max() + 1   # ties: the first maximum
    assert po.sample(lg2, 0.0, 1.0) == 10


def test_accept_match_brute_force():
    rng = np.random.default_rng(4)
    V, n = 50, 5
    for trial in range(100):
        lg = rng.standard_normal((n, V)).astype(np.float32) * 2
        batch = rng.integers(0, V, n).astype(np.int32)
        if trial % 2:   # drafts that the greedy rows would pick
            batch[1:] = np.argmax(lg[:-1], 1)
        u = rng.random(n)
        T = 0.0 if trial % 3 == 0 else 0.8
        out, kept = po.accept_match(lg, batch, T, 0.9, 0, 1024, u)
        want = []
        for i in range(n):
            y = po.sample(lg[i], T, 0.9, 0, 1024, float(u[i]))
            want.append(y)
            if not (i + 1 < n and y == batch[i + 1]):
                break
        assert list(out) == want and kept == len(want)


def test_textbook_rule_output_distribution_is_p():
    """P(first emitted token = x) equals p_0(x) exactly in the limit: integrated over a grid of uniforms."""
    rng = np.random.default_rng(9)
    V, k = 6, 2
    target = (rng.standard_normal((k + 1, V)) * 1.5).astype(np.float32)
    draft = (target[:k] + rng.standard_normal((k, V)) * 0.8).astype(np.float32)
    T, top_p = 0.9, 1.0
    p0 = po.nucleus_probs(target[0], T, top_p)
    g = (np.arange(48) + 0.5) / 48
    counts = np.zeros(V)
    for ud in g:
        for ua in g:
            for ur in g[::2]:
                out = po.accept_textbook(target, draft, T, top_p, False, [ud, 0.5], [ua, 0.5], ur)
                counts[out[0]] += 1
    freq = counts / counts.sum()
    assert np.abs(freq - p0).max() < 0.03


def test_textbook_rule_chi_square_and_greedy():
    rng = np.random.default_rng(10)
    V, k = 8, 3
    target = (rng.standard_normal((k + 1, V)) * 1.2).astype(np.float32)
    draft = (target[:k] + rng.standard_normal((k, V)) * 0.5).astype(np.float32)
    p0 = po.nucleus_probs(target[0], 0.7, 0.95)
    N = 20000
    us = rng.random((N, 2 * k + 1)).astype(np.float32)
    counts = np.zeros(V)
    for i in range(N):
        out = po.accept_textbook(target, draft, 0.7, 0.95, False, us[i, :k], us[i, k:2 * k], us[i, -1])
        counts[out[0]] += 1
    expected = p0 * N
    m = expected > 0
    assert counts[~m].sum() == 0
    chi2 = float(((counts[m] - expected[m]) ** 2 / expected[m]).sum())
    assert chi2 < 40.0   # dof <= 7: far above the 0.999 quantile (24.3) would flag a wrong rule
    # greedy: drafts accepted while argmaxes agree, then the target's argmax
    draft_g = target[:k].copy()
    draft_g[1] = np.roll(target[1], 1)
    out = po.accept_textbook(target, draft_g, 0.7, 0.95, True, [0] * k, [0] * k, 0)
    assert list(out) == [int(np.argmax(target[0])), int(np.argmax(target[1]))]


# ---------------------------------------------------------------- the presence penalty and stop tokens
def test_accept_match_ex_without_penalty_or_stops_is_accept_match():
    rng = np.random.default_rng(71)
    x = (rng.standard_normal((5, 500)) * 2).astype(np.float32)
    u = rng.random(5)
    for t in (0.0, 0.8):
        for trial in range(6):
            batch = np.concatenate([[3], rng.integers(0, 500, 4)]).astype(np.int32)
            if trial % 2:   # drafts the rows sample: some stand
                batch[1:] = [po.sample(x[i], t, 0.95, 0, 1024, u[i]) for i in range(4)]
            a, ka = po.accept_match(x, batch, t, 0.95, 0, 1024, u)
            b, kb, lg = po.accept_match_ex(x, batch, t, 0.95, 0, 1024, u)
            assert list(a) == list(b) and ka == kb
            assert np.array_equal(lg, x)   # no penalty: the rows untouched


def test_presence_penalty_closed_form_greedy():
    """geode.cpp:247-255: every seen token loses the penalty once before the row is sampled; a draft that stood joins
    the seen tokens of the rows after it"""
    V = 16
    x = np.zeros((3, V), np.float32)
    x[:, 5] = 3.0   # the favourite of every row
    x[:, 9] = 2.5
    x[:, 2] = 2.0
    # nothing seen: rows 0.. sample 5; with 5 seen (penalty 1: 5 -> 2.0 < 2.5), row 0 samples 9
    out, kept, lg = po.accept_match_ex(x, [1, 9, 2], 0.0, 1.0, seen=[5], presence_penalty=1.0)
    # row 0: argmax of (5: 2.0, 9: 2.5, 2: 2.0) = 9 = draft 1, stands; row 1: 5 and 9 seen: (2.0, 1.5, 2.0): the first
    # argmax is token 2 = draft 2, stands; row 2: the last row, sampled: 5, 9, 2 all seen -> (2.0, 1.5, 1.0) -> 5
    assert list(out) == [9, 2, 5] and kept == 3
    assert lg[0, 5] == 2.0 and lg[0, 9] == 2.5                     # row 0: only the seen token
    assert lg[1, 5] == 2.0 and lg[1, 9] == 1.5 and lg[1, 2] == 2.0   # row 1: + the stood draft 9
    assert lg[2, 2] == 1.0                                          # row 2: + the stood draft 2
    # a token that is both seen and a stood draft again loses the penalty once: row 0 samples 5 (5: 3.0 > 9: 2.25),
    # the draft 5 stands; rows 1 and 2 lose 0.25 at 9 and at 5, once each
    out, kept, lg = po.accept_match_ex(x, [1, 5, 5], 0.0, 1.0, seen=[9], presence_penalty=0.25)
    assert list(out) == [5, 5, 5] and kept == 3
    assert lg[1, 5] == np.float32(2.75) and lg[1, 9] == np.float32(2.25)
    assert lg[2, 5] == np.float32(2.75) and lg[2, 9] == np.float32(2.25)


def test_stop_token_draft_does_not_stand():
    """geode.cpp:333: a draft equal to the sampled token stands only if it is no stop token; the stop token is then
    the token emitted (and the answer ends there)"""
    V = 8
    x = np.zeros((3, V), np.float32)
    x[0, 4] = x[1, 6] = x[2, 1] = 5.0
    out, kept, _ = po.accept_match_ex(x, [0, 4, 6], 0.0, 1.0)
    assert list(out) == [4, 6, 1] and kept == 3
    out, kept, _ = po.accept_match_ex(x, [0, 4, 6], 0.0, 1.0, stop=[6])
    assert list(out) == [4, 6] and kept == 2
    out, kept, _ = po.accept_match_ex(x, [0, 4, 6], 0.0, 1.0, stop=[4, 7])
    assert list(out) == [4] and kept == 1
