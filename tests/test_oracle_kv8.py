"""The CPU oracle's int8 KV cache (attend<int8_t>, engine/src/model.cpp:3756-3792, :3929-3972): quant_kv_row
against its defining properties, and the int8 model against the reference's stated invariants (a row's logits do
not depend on its batch, model.hpp:189-193; a tree row is the chain through its ancestors; keep = a verify of the
kept prefix) and against the fp16 cache it quantizes."""
import numpy as np
import pytest

import pyoracle as po
from model_helpers import SMALL, SMALL_ROUTER_SIGMA, rel_err, tree_parents

CTX = 90
SMALL8 = dict(SMALL, kv_int8=1)


def test_quant_kv_row_properties():
    rng = np.random.default_rng(3)
    for n in (64, 256):
        for _ in range(20):
            x = (rng.standard_normal(n) * rng.uniform(0.01, 50)).astype(np.float32)
            q, s = po.quant_kv_row(x)
            amax = np.abs(x).max()
            assert s == np.float32(amax) / np.float32(127)                       # scale = amax / 127
            i = int(np.argmax(np.abs(x)))
            assert q[i] == (127 if x[i] > 0 else -127)                           # the largest maps to +-127
            assert np.abs(q.astype(np.int32)).max() <= 127
            assert np.all(np.sign(q) * np.sign(x) >= 0)                          # signs kept
            err = np.abs(q.astype(np.float64) * s - x)
            assert err.max() <= 0.5 * s * (1 + 1e-5) + 1e-7 * amax               # nearest level
    q, s = po.quant_kv_row(np.zeros(64, np.float32))
    assert s == 0.0 and not q.any()                                              # a zero row
    # ties go to the even level: x * (127 / amax) = k + 1/2 exactly (amax = 127: the factor is 1)
    x = np.array([127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5] + [0.0] * 57, np.float32)
    q, s = po.quant_kv_row(x)
    assert list(q[:7]) == [127, 2, 4, -2, -4, 0, 0] and s == 1.0


@pytest.fixture(scope="module")
def om8():
    return po.Model(SMALL8, seed=7, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)


def test_int8_batched_equals_one_at_a_time(om8):
    toks = np.array([3, 141, 59, 265, 358], np.int32)
    om8.position = CTX
    batched = om8.verify(toks)
    om8.position = CTX
    rows = [om8.verify(toks[i:i + 1])[0] for i in range(toks.size)]
    assert np.array_equal(batched.view(np.uint32), np.array(rows).view(np.uint32))


def test_int8_tree_row_is_the_chain_of_its_ancestors(om8):
    parents = tree_parents((2, 2))
    toks = (np.arange(parents.size) * 37 + 11) % SMALL["vocab"]
    om8.position = CTX
    tree = om8.verify(toks, parents)
    for leaf in (3, 6):
        path = [leaf]
        while parents[path[-1]] >= 0:
            path.append(int(parents[path[-1]]))
        path = path[::-1]
        om8.position = CTX
        chain = om8.verify(toks[path])
        assert np.array_equal(tree[leaf].view(np.uint32), chain[-1].view(np.uint32))


def test_int8_keep_equals_verify_of_the_kept_prefix(om8):
    parents = tree_parents((2, 2))
    toks = (np.arange(parents.size) * 53 + 5) % SMALL["vocab"]
    path = np.array([0, 2, 6], np.int32)
    om8.position = CTX
    om8.verify(toks, parents)
    om8.keep(3, path)
    nxt = om8.verify(np.array([77], np.int32))
    om8.position = CTX
    om8.verify(toks[path])
    again = om8.verify(np.array([77], np.int32))
    assert np.array_equal(nxt.view(np.uint32), again.view(np.uint32))


def test_int8_close_to_the_fp16_cache(om8):
    """the same weights and context (N(0, 1) keys and values, here quantized per row to int8, there rounded to fp16):
    logits within a few percent. A dropped K or V scale, or a scale applied twice, is off by orders of magnitude."""
    om16 = po.Model(SMALL, seed=7, router_sigma=SMALL_ROUTER_SIGMA, ctx=CTX)
    toks = np.array([3, 141, 59, 265, 358], np.int32)
    om8.position = CTX
    om16.position = CTX
    a, b = om8.verify(toks), om16.verify(toks)
    assert rel_err(a, b) < 5e-2
