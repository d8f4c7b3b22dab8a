"""The generate loop's restatement (tests/spec_loop.py) on the CPU oracle alone: the speculative loop, with the MTP
layer's drafts or with drafts taken from the answer, emits the one-token-at-a-time answer (engine/src/geode.cpp:221-224),
greedy and stochastic with the presence penalty and a stop token; and a planted slip in the loop (a stood draft's
uniform not consumed) is caught. The GPU's loop is compared with this one in tests/test_gpu_spec_loop.py."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL
from spec_loop import Log, OracleBackend, Uniforms, generate

CTX = 60
CFG = dict(SMALL, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
           gdn_layers=[1, 0, 1], mtp=1, max_ctx=160)
SAMPLING = {"greedy": dict(T=0.0, top_p=1.0, penalty=0.0), "stochastic": dict(T=0.7, top_p=0.95, penalty=0.3)}


@pytest.fixture(scope="module")
def om():
    return po.Model(CFG, seed=17, router_sigma=1.0 / np.sqrt(CFG["hidden"]), ctx=CTX)


def _run(om, states, mode, **kw):
    for l, (conv, S) in states.items():
        om.tensor(po.GDN_CONV_ST, l)[0][:] = conv
        om.tensor(po.GDN_S, l)[0][:] = S
    om.position = CTX
    log = Log()
    prompt = np.array([5, 77, 300, 12, 9], np.int32)
    toks = generate(OracleBackend(om, mode=1), prompt, 32, Uniforms(99), kmax=5, pmin=0.0, log=log,
                    **SAMPLING[mode], **kw)
    return toks, log


def _replacer(answer, seed):
    rng = np.random.default_rng(seed)

    def replace(out, drafts):
        return [int(answer[len(out) + j]) if len(out) + j < len(answer) and rng.random() < 0.7
                else int(rng.integers(0, 64)) for j in range(len(drafts))]
    return replace


@pytest.mark.parametrize("mode", ["greedy", "stochastic"])
def test_speculative_loop_is_the_one_token_answer(om, mode):
    states = {l: (om.tensor(po.GDN_CONV_ST, l)[0].copy(), om.tensor(po.GDN_S, l)[0].copy()) for l in (0, 2)}
    answer, _ = _run(om, states, mode, spec=False)
    stop = ()
    if mode == "stochastic":   # a stop token first seen at index >= 20: the answer ends there
        k = next(k for k in range(20, len(answer)) if answer[k] not in answer[:k])
        stop = (answer[k],)
        answer = answer[:k + 1]
        assert _run(om, states, mode, spec=False, stop=stop)[0] == answer
    mtp, _ = _run(om, states, mode, stop=stop)
    informed, log = _run(om, states, mode, stop=stop, replace_drafts=_replacer(answer, 3))
    assert mtp == answer
    assert informed == answer
    assert len(set(log.kept)) >= 3   # drafts stood to several depths


def test_a_slip_in_the_loop_is_caught(om, monkeypatch):
    """the loop with a stood draft's uniform left unconsumed (planted in the uniform stream) no longer emits the
    one-token answer: the comparison above can fail"""
    states = {l: (om.tensor(po.GDN_CONV_ST, l)[0].copy(), om.tensor(po.GDN_S, l)[0].copy()) for l in (0, 2)}
    answer, _ = _run(om, states, "stochastic", spec=False)
    take = Uniforms.take
    calls = {"n": 0}

    def slipped(self, n):
        calls["n"] += 1
        if calls["n"] != 4:   # the fourth take (a stood draft's or a next token's) is skipped
            take(self, n)
    monkeypatch.setattr(Uniforms, "take", slipped)
    toks, _ = _run(om, states, "stochastic", replace_drafts=_replacer(answer, 3))
    assert toks != answer
