"""The reference's generate loop (engine/src/geode.cpp:215-384, with read_prompt's MTP pass, :70-151) restated over a
backend, for the loop tests: the prompt verified and its MTP rows filled, the first token sampled from the prompt's
last row, then per step the MTP drafts (draft, then draft_next while confident, geode.cpp:301-317), the batch [tok,
drafts] verified, sample-and-match over its rows (each row sampled with the next uniform of the stream, a draft
standing while it is what its row samples and is no stop token, geode.cpp:318-350), verify_keep of the rows that
stood, and the MTP bookkeeping for the next step (mtp_n = kept, mtp_pos = the batch's first position, the hidden rows
the verify's). Without drafting (spec=False) it is the one-token-at-a-time loop (geode.cpp:376-380). A draft never
changes the answer: every emitted token is sampled from its own verified logits with its own uniform.

Two backends: `GpuBackend` (the library through its C ABI: gv_verify, gv_verify_keep, gv_model_mtp_fill,
gv_model_draft_chain, gv_accept_match_ex) and `OracleBackend` (the CPU oracle's Model and accept_match_ex).
`replace_drafts` lets a test swap drafts for tokens it knows (an answer computed before), so that with random weights
drafts still stand and the keep / stop paths run: the tokens drafted never change what is emitted.

Test infrastructure only."""
import numpy as np

import pyoracle as po


class Uniforms:
    """a seeded stream of U[0, 1) doubles, taken one per sampled row in the order the loop samples"""

    def __init__(self, seed, n=4096):
        self.u = np.random.default_rng(seed).random(n)
        self.i = 0

    def peek(self, n):
        return self.u[self.i:self.i + n]

    def take(self, n):
        self.i += n


class GpuBackend:
    def __init__(self, gv, gm):
        self.gv, self.gm = gv, gm

    @property
    def position(self):
        return self.gm.position

    def verify(self, toks):
        return self.gm.verify(np.asarray(toks, np.int32))

    def keep(self, kept):
        self.gm.keep(kept)

    def hidden(self):
        return self.gm.hidden()

    def mtp_fill(self, toks, pos, hidden):
        self.gm.mtp_fill(np.asarray(toks, np.int32), pos, hidden)

    def drafts(self, toks, pos, hidden, kmax, pmin):
        d, _ = self.gm.draft_chain(np.asarray(toks, np.int32), pos, kmax, pmin, hidden)
        return [int(x) for x in d]

    def accept(self, logits, batch, T, top_p, u, seen, penalty, stop):
        out, kept, _ = self.gv.accept_match_ex(logits, batch, T, top_p, u=u, seen=seen, presence_penalty=penalty,
                                               stop=stop)
        return [int(x) for x in out], kept


class OracleBackend:
    def __init__(self, om, mode=0):
        self.om, self.mode = om, mode

    @property
    def position(self):
        return self.om.position

    def verify(self, toks):
        return self.om.verify(np.asarray(toks, np.int32), mode=self.mode)

    def keep(self, kept):
        self.om.keep(kept)

    def hidden(self):
        return self.om.hidden()

    def mtp_fill(self, toks, pos, hidden):
        self.om.mtp(np.asarray(toks, np.int32), pos, hidden, mode=self.mode, logits=False)

    def drafts(self, toks, pos, hidden, kmax, pmin):
        """geode.cpp:301-317: draft, then draft_next while the last probability is at least pmin"""
        d, p, _ = self.om.draft(np.asarray(toks, np.int32), pos, hidden, mode=self.mode)
        out = [d]
        q = pos + len(toks)
        while len(out) + 1 < kmax and p >= pmin and self.om.position + len(out) + 2 < self.om.cfg["max_ctx"]:
            d2, p, _ = self.om.draft_next(out[-1], q, mode=self.mode)
            if p < pmin:
                break
            out.append(d2)
            q += 1
        return out

    def accept(self, logits, batch, T, top_p, u, seen, penalty, stop):
        out, kept, _ = po.accept_match_ex(logits, batch, T, top_p, u=u, seen=seen, presence_penalty=penalty,
                                          stop=stop)
        return [int(x) for x in out], kept


class Log:
    """what a run did: the steps' batch lengths and kept rows (to show the drafts stood and were taken back)"""

    def __init__(self):
        self.batches, self.kept = [], []


def generate(be, prompt, max_tokens, uniforms, T=0.0, top_p=1.0, penalty=0.0, stop=(), spec=True, kmax=5,
             pmin=0.8, replace_drafts=None, fail_at=None, log=None):
    """The answer's tokens. fail_at = (step, handler): at that verify step the handler is called with (backend, batch,
    the answer so far) instead of the backend's verify and returns (backend to go on with, the batch's logits) -- the
    fallback tests' hook."""
    ctx = be.om.cfg["max_ctx"] if isinstance(be, OracleBackend) else be.gm.cfg["max_ctx"]
    log = log if log is not None else Log()
    prompt = [int(t) for t in prompt]
    p0 = be.position
    logits = be.verify(prompt)
    prev = None
    if spec:   # read_prompt's MTP rows: hidden row r with the prompt's token r + 1, at MTP position p0 + r
        hid = be.hidden()
        if len(prompt) > 1:
            be.mtp_fill(prompt[1:], p0, hid[:len(prompt) - 1])
        prev = hid[len(prompt) - 1:len(prompt)]
    seen = []
    out = []

    def sample_one(row):
        """Sampler::sample of one row with the presence penalty (geode.cpp:247-255), one uniform"""
        got, _ = be.accept(row[None, :], [0], T, top_p, uniforms.peek(1), list(seen), penalty, ())
        uniforms.take(1)
        tok = got[0]
        if penalty != 0.0 and tok not in seen:
            seen.append(tok)
        return tok

    tok = sample_one(logits[-1])
    mtp_tok, mtp_n, mtp_pos, mtp_hidden = [0] * 32, 1, be.position - 1, prev
    step = 0
    while True:
        out.append(tok)
        if tok in stop:
            break
        if len(out) >= max_tokens or be.position + 1 >= ctx:
            break
        if spec and be.position + 2 < ctx:
            mtp_tok[mtp_n - 1] = tok
            drafts = be.drafts(mtp_tok[:mtp_n], mtp_pos, mtp_hidden, kmax, pmin)
            drafts = drafts[:max(0, min(len(drafts), ctx - be.position - 2))]
            if replace_drafts is not None:
                drafts = replace_drafts(out, drafts)
            batch = [tok] + drafts
            n = len(batch)
            if fail_at is not None and step == fail_at[0]:
                be, lg = fail_at[1](be, batch, out)
            else:
                lg = be.verify(batch)
            step += 1
            P = be.position - n
            u = uniforms.peek(n)
            emitted, kept = be.accept(lg, batch, T, top_p, u, list(seen), penalty, stop)
            log.batches.append(n)
            log.kept.append(kept)
            # the rows sampled, in order: the stood drafts, then the next token (geode.cpp:327-350); the last emitted
            # token is always the next one, so kept = len(emitted) (tok and the drafts that stood)
            assert kept == len(emitted)
            stood = emitted[:-1]
            stop_now = False
            for i, y in enumerate(stood):
                uniforms.take(1)
                if penalty != 0.0 and y not in seen:
                    seen.append(y)
                out.append(y)
                mtp_tok[i] = y
                if len(out) >= max_tokens or P + i + 1 + 1 >= ctx:
                    stop_now = True
                    break
            if stop_now:   # the answer ends on a stood draft: taken back and left pending (geode.cpp:351-361)
                be.keep(i + 1)
                break
            nxt = emitted[-1]
            uniforms.take(1)
            if penalty != 0.0 and nxt not in seen:
                seen.append(nxt)
            mtp_tok[len(stood)] = nxt
            if kept < n:
                be.keep(kept)
            tok = nxt
            mtp_n, mtp_pos, mtp_hidden = kept, P, None
            continue
        lg = be.verify([tok])
        tok = sample_one(lg[0])
    return out
