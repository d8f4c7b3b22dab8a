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
