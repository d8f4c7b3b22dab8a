"""The speculative loop end to end on the GPU (engine/src/geode.cpp:215-384, restated in tests/spec_loop.py): MTP
drafts (gv_model_draft_chain) -> gv_verify -> sample-and-match with the presence penalty and stop tokens
(gv_accept_match_ex) -> gv_verify_keep, for 64 emitted tokens, against the same loop on the CPU oracle and against
one-token-at-a-time decoding on both. The reference states the invariant (geode.cpp:221-224, :270-275): the answer is
the one-token-at-a-time answer, whatever the drafts.

Models: the real model's shape at test size (Gated DeltaNet and attention layers, the MTP layer) and C4's width
(hidden 2048, 256 experts, 16 / 2 heads of 256, the 151,936-token vocabulary) with an MTP layer. The exact path on
the GPU against the oracle's exact mode (their logits agree to ~1e-6, so tokens agree away from sampling
boundaries); the int8 path on the GPU against itself one token at a time. Greedy and seeded stochastic (T 0.7, top-p
0.95, presence penalty 0.3, a stop token), the uniforms one per sampled row from a seeded stream.

With random weights an MTP draft rarely equals the sampled token, so each answer is also run with drafts replaced by
tokens of the known answer (70% of them right, seeded): the drafts then stand or fall at every depth and the keep,
stop and max_tokens paths run; the answer must not change. A run with the MTP's own drafts is the composition as
the reference runs it.

Fallback identity (the reference's backend seam: a failed backend call returns nonzero with a message and the
engine's CPU path takes the step, engine/src/model.cpp:1557-1563, geode.cpp:318-323): at the third verify the GPU
is handed a batch it refuses (a token outside the vocabulary); the refusal must leave the GPU model's state as it
was, and the answer must be the same whether the loop then goes on on the CPU (the oracle brought to the
conversation) or on the GPU."""
import os

import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, adopt_oracle_model
from spec_loop import GpuBackend, Log, OracleBackend, Uniforms, generate

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

CTX = 90
REAL = dict(SMALL, n_layers=3, gdn_k_heads=2, gdn_v_heads=4, gdn_k_dim=32, gdn_v_dim=32, conv_kernel=4,
            gdn_layers=[1, 0, 1], mtp=1, max_ctx=256)
C4W = dict(hidden=2048, vocab=151936, n_layers=2, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
           n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=512, max_rows=17, mtp=1)
C4W_CTX = 400
N_TOKENS = 64
SAMPLING = {"greedy": dict(T=0.0, top_p=1.0, penalty=0.0),
            "stochastic": dict(T=0.7, top_p=0.95, penalty=0.3)}


class Setup:
    """an oracle model and GPU models of the same weights (exact path, int8 path), restartable at the context"""

    def __init__(self, gv, cfg, ctx, seed):
        po.lib.orc_set_threads(min(16, os.cpu_count() or 1))
        self.gv, self.cfg, self.ctx = gv, cfg, ctx
        self.om = po.Model(cfg, seed=seed, router_sigma=1.0 / np.sqrt(cfg["hidden"]), ctx=ctx, fast=cfg["hidden"] > 256)
        self.gx = gv.VerifyModel(dict(cfg, exact=1))
        adopt_oracle_model(self.gx, self.om, ctx)
        self.g8 = gv.VerifyModel(cfg)
        adopt_oracle_model(self.g8, self.om, ctx)
        # the Gated DeltaNet layers' states at the context, to start every run from
        gdn = cfg.get("gdn_layers", ())
        self.states = {l: (self.om.tensor(po.GDN_CONV_ST, l)[0].copy(), self.om.tensor(po.GDN_S, l)[0].copy())
                       for l in range(len(gdn)) if gdn[l]}

    def restart(self):
        """every model at the context with its initial states"""
        g = self.gv
        for l, (conv, S) in self.states.items():
            self.om.tensor(po.GDN_CONV_ST, l)[0][:] = conv
            self.om.tensor(po.GDN_S, l)[0][:] = S
            for gm in (self.gx, self.g8):
                gm.adopt(g.GDN_CONV_ST, conv, layer=l)
                gm.adopt(g.GDN_S, S, layer=l)
        self.om.position = self.ctx
        self.gx.position = self.ctx
        self.g8.position = self.ctx

    def close(self):
        self.gx.close()
        self.g8.close()
        po.lib.orc_set_threads(1)


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


@pytest.fixture(scope="module")
def real(gv):
    s = Setup(gv, REAL, CTX, 17)
    yield s
    s.close()


def _prompt(cfg, seed):
    return np.random.default_rng(seed).integers(0, cfg["vocab"], 6).astype(np.int32)


def _stop_for(answer):
    """a stop token that first appears at index >= 40 of the answer (its answer then ends there), or none"""
    for k in range(40, len(answer)):
        if answer[k] not in answer[:k]:
            return (int(answer[k]),), answer[:k + 1]
    return (), answer


def _replacer(answer, seed):
    """drafts replaced by the answer's next tokens, each right with probability 0.7"""
    rng = np.random.default_rng(seed)

    def replace(out, drafts):
        got = []
        for j in range(len(drafts)):
            i = len(out) + j
            right = i < len(answer) and rng.random() < 0.7
            got.append(int(answer[i]) if right else int(rng.integers(0, 64)))
        return got
    return replace


def _run(s, be, prompt, mode, stop=(), spec=True, replace=None, fail_at=None, pmin=0.0):
    s.restart()
    log = Log()
    toks = generate(be, prompt, N_TOKENS, Uniforms(1234), stop=stop, spec=spec, kmax=5, pmin=pmin,
                    replace_drafts=replace, fail_at=fail_at, log=log, **SAMPLING[mode])
    return toks, log


def _loop_identity(s, mode, prompt):
    om = s.om
    oracle = OracleBackend(om, mode=1)
    gpu = GpuBackend(s.gv, s.gx)
    answer, _ = _run(s, oracle, prompt, mode, spec=False)
    stop, answer_stop = _stop_for(answer) if mode == "stochastic" else ((), answer)
    if stop:
        answer, _ = _run(s, oracle, prompt, mode, stop=stop, spec=False)
        assert answer == answer_stop
    runs = {"gpu, one at a time": _run(s, gpu, prompt, mode, stop, spec=False),
            "gpu, MTP drafts": _run(s, gpu, prompt, mode, stop),
            "gpu, drafts from the answer": _run(s, gpu, prompt, mode, stop, replace=_replacer(answer, 5)),
            "oracle, drafts from the answer": _run(s, oracle, prompt, mode, stop, replace=_replacer(answer, 5))}
    print(f"\n{mode}: answer of {len(answer)} tokens (stop {stop})", flush=True)
    for name, (toks, log) in runs.items():
        steps = len(log.batches)
        stood = sum(k - 1 for k in log.kept)
        print(f"  {name}: {len(toks)} tokens, {steps} verify steps, batches {sorted(set(log.batches))}, drafts stood "
              f"{stood} of {sum(b - 1 for b in log.batches)}, kept counts {sorted(set(log.kept))}", flush=True)
        first = next((i for i, (a, b) in enumerate(zip(toks, answer)) if a != b), None)
        assert toks == answer, f"{mode}, {name}: differs from the one-token-at-a-time answer at token {first}"
    replaced = runs["gpu, drafts from the answer"][1]
    assert len(set(replaced.kept)) >= 3, "the drafts from the answer should stand to several depths"
    return answer


@pytest.mark.parametrize("mode", ["greedy", "stochastic"])
def test_loop_is_the_one_token_answer(real, mode):
    _loop_identity(real, mode, _prompt(REAL, 3))


def test_int8_loop_equals_its_one_token_answer(real):
    """the int8 path on the GPU: the speculative loop (drafts from its own one-token answer) gives that answer"""
    gpu = GpuBackend(real.gv, real.g8)
    prompt = _prompt(REAL, 4)
    for mode in ("greedy", "stochastic"):
        answer, _ = _run(real, gpu, prompt, mode, spec=False)
        toks, log = _run(real, gpu, prompt, mode, replace=_replacer(answer, 9))
        mtp, _ = _run(real, gpu, prompt, mode)
        print(f"\nint8 {mode}: {len(answer)} tokens; drafts stood {sum(k - 1 for k in log.kept)} in "
              f"{len(log.batches)} steps", flush=True)
        assert toks == answer and mtp == answer, f"int8 {mode}: the loop's answer differs from one token at a time"


def _refuse_then(s, prompt, go_on):
    """a fail_at handler: the batch with a token outside the vocabulary is refused and changes nothing; the step
    (and the rest) then runs on the CPU oracle brought to the conversation, or again on the GPU"""
    gv, gm, om, cfg = s.gv, s.gx, s.om, s.cfg

    def handler(be, batch, out):
        pos0 = gm.position
        bad = list(batch)
        bad[-1] = cfg["vocab"] + 7
        with pytest.raises(gv.GeodeError, match="token out of range"):
            gm.verify(np.asarray(bad, np.int32))
        assert gm.position == pos0, "a refused verify moved the position"
        if go_on == "gpu":
            return be, be.verify(batch)
        # the CPU path: the oracle reads the conversation the GPU model holds (the prompt and the answer so far
        # but its pending last token), with the MTP rows read_prompt would fill, then verifies the batch
        conv = [int(t) for t in prompt] + out[:-1]
        nxt = conv[1:] + [out[-1]]
        om.position = s.ctx
        for c0 in range(0, len(conv), cfg["max_rows"]):
            om.verify(np.asarray(conv[c0:c0 + cfg["max_rows"]], np.int32), mode=1)
            hid = om.hidden()
            om.mtp(np.asarray(nxt[c0:c0 + hid.shape[0]], np.int32), s.ctx + c0, hid, mode=1, logits=False)
        assert om.position == pos0
        oracle = OracleBackend(om, mode=1)
        return oracle, oracle.verify(batch)
    return handler


@pytest.mark.parametrize("go_on", ["cpu", "gpu"])
def test_fallback_after_a_refused_verify(real, go_on):
    prompt = _prompt(REAL, 3)
    mode = "stochastic"
    gpu = GpuBackend(real.gv, real.gx)
    answer, _ = _run(real, OracleBackend(real.om, mode=1), prompt, mode, spec=False)
    stop, answer = _stop_for(answer)
    handler = _refuse_then(real, prompt, go_on)

    def fail(be, batch, out):
        return handler(be, batch, out)
    toks, log = _run(real, gpu, prompt, mode, stop, replace=_replacer(answer, 5), fail_at=(2, fail))
    print(f"\nfallback ({go_on} after the refusal at the third verify): {len(toks)} tokens, "
          f"{len(log.batches)} steps", flush=True)
    assert toks == answer, "the answer changed after the refused verify"


def test_loop_at_c4_width(gv):
    """C4's width (2 layers + the MTP layer, the full vocabulary): the GPU's loop is the oracle's one-token answer"""
    s = Setup(gv, C4W, C4W_CTX, 23)
    try:
        prompt = _prompt(C4W, 6)
        for mode in ("greedy", "stochastic"):
            answer, _ = _run(s, OracleBackend(s.om, mode=1), prompt, mode, spec=False)
            stop, answer = _stop_for(answer) if mode == "stochastic" else ((), answer)
            gpu = GpuBackend(gv, s.gx)
            toks, log = _run(s, gpu, prompt, mode, stop, replace=_replacer(answer, 7))
            mtp, mlog = _run(s, gpu, prompt, mode, stop)
            print(f"\nC4 width, {mode}: {len(answer)} tokens; drafts from the answer stood "
                  f"{sum(k - 1 for k in log.kept)} in {len(log.batches)} steps; MTP drafts stood "
                  f"{sum(k - 1 for k in mlog.kept)} in {len(mlog.batches)} steps", flush=True)
            assert toks == answer, f"C4 width {mode}: the loop's answer differs from the one-token answer"
            assert mtp == answer, f"C4 width {mode}: the MTP loop's answer differs from the one-token answer"
    finally:
        s.close()
