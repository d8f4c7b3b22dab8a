"""C2 at its own size: 1024 seeded trials per mode of the acceptance step on the GPU
against the oracle. Vocabulary 151,936, k = 4 chain drafts; target logits fp32 N(0, 3), draft logits the target
rows plus N(0, 0.5); T = 0.7, top-p 0.95; seeded fp32 uniforms for each draft's sample, its acceptance and the
residual / bonus draw (trial t: seeds 1000 + t).

* textbook rule (min(1, p/q) acceptance, residual resampling from max(0, p - q), a bonus token when all stand):
  greedy and stochastic, against po.accept_textbook;
* sample-and-match, the reference's own rule (engine/src/geode.cpp:318-374), with the drafts the argmax of the
  draft rows (the reference drafts greedily), greedy (T = 0) and stochastic, against po.accept_match.

Outputs must be identical except at near-ties: a trial whose tokens differ passes only if the oracle's own answer
changes when its uniforms move by 1e-6 (relative), i.e. a uniform sits on a decision boundary to within the GPU's
summation-order differences. Mismatch and near-tie counts are printed."""
import concurrent.futures

import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu

V, K, T, TOP_P = 151936, 4, 0.7, 0.95
TRIALS = 1024


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def _trial(t):
    seed = 1000 + t
    target = po.normal(seed * 4, (K + 1) * V, 3.0).reshape(K + 1, V)
    draft = target[:K] + po.normal(seed * 4 + 1, K * V, 0.5).reshape(K, V)
    u = po.uniform(seed * 4 + 2, 2 * K + 1)
    return target, draft, u[:K], u[K:2 * K], np.float32(u[2 * K])


def _run(fn, items, workers=16):
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:   # (ctypes calls release the GIL)
        return list(ex.map(fn, items))


def _chunks(make, gpu, cpu, chunk=64):
    """(GPU results, oracle results) over all trials, a chunk of inputs in memory at a time"""
    got, want = [], []
    for t0 in range(0, TRIALS, chunk):
        items = _run(make, range(t0, min(TRIALS, t0 + chunk)))
        got += [gpu(a) for a in items]
        want += _run(cpu, items)
    return got, want


def _check(mode, got, want, unstable):
    bad = [t for t in range(TRIALS) if list(got[t]) != list(want[t])]
    ties = [t for t in bad if unstable(t)]
    print(f"C2 {mode}: {TRIALS} trials, {len(bad)} mismatches, {len(ties)} of them near-ties "
          f"(mean tokens emitted {np.mean([len(w) for w in want]):.3f})", flush=True)
    assert bad == ties, f"{mode}: trials {sorted(set(bad) - set(ties))[:10]} differ with no near-tie"


@pytest.mark.parametrize("greedy", [False, True])
def test_textbook_1024_trials(gv, greedy):
    got, want = _chunks(_trial, lambda a: gv.accept_textbook(a[0], a[1], T, TOP_P, greedy, a[2], a[3], a[4]),
                        lambda a: po.accept_textbook(a[0], a[1], T, TOP_P, greedy, a[2], a[3], a[4]))

    def unstable(t):
        tg, dr, ud, ua, ur = _trial(t)
        if greedy:   # the argmaxes: a top-2 gap of an ulp or so
            s = np.sort(np.concatenate([tg, dr]), axis=1)
            return bool(((s[:, -1] - s[:, -2]) <= 1e-6 * np.abs(s[:, -1])).any())
        base = list(want[t])
        for f in (1 + 1e-6, 1 - 1e-6):
            alt = po.accept_textbook(tg, dr, T, TOP_P, greedy, (ud * f).astype(np.float32),
                                     (ua * f).astype(np.float32), np.float32(ur * f))
            if list(alt) != base:
                return True
        return False

    _check("textbook greedy" if greedy else "textbook stochastic", got, want, unstable)


def _match_trial(t):
    tg, dr, ud, ua, ur = _trial(t)
    batch = np.concatenate([[t % V], np.argmax(dr, axis=1)]).astype(np.int32)   # the drafts: argmax of q
    return tg, batch, np.concatenate([ua, [ur]]).astype(np.float64)


@pytest.mark.parametrize("greedy", [False, True])
def test_sample_and_match_1024_trials(gv, greedy):
    temp = 0.0 if greedy else T
    got, want = _chunks(_match_trial, lambda a: gv.accept_match(a[0], a[1], temp, TOP_P, 0, 1024, a[2]),
                        lambda a: po.accept_match(a[0], a[1], temp, TOP_P, 0, 1024, a[2]))

    def unstable(t):
        tg, b, u = _match_trial(t)
        for f in (1 + 1e-6, 1 - 1e-6):
            alt = po.accept_match(tg, b, temp, TOP_P, 0, 1024, u * f)
            if list(alt[0]) != list(want[t][0]):
                return True
        return False

    _check("match greedy" if greedy else "match stochastic", [g[0] for g in got], [w[0] for w in want], unstable)
    for t in range(TRIALS):
        assert got[t][1] == want[t][1] or unstable(t)
