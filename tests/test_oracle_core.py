"""The oracle pinned (CPU): against the reference's own outputs (tests/golden/ref_vectors.npz, written by
tests/golden/make_golden.py from oracle/_ref), against oracle/_ref directly where it is built, and against closed
forms, invariants and brute force chosen so that a dropped term, a wrong sign or index fails one of them."""
import math
import os

import numpy as np
import pytest

import pyoracle as po

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
P = po._ptr


@pytest.fixture(scope="module")
def ref():
    """the reference built here from its own sources (oracle/_ref), loaded only by the CPU tests that use it: it is
    never shipped to or loaded on the GPU box"""
    r = po.load_ref()
    if r is None:
        pytest.skip("oracle/_ref not built here")
    return r


def u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- E4M3
def test_e4m3_matches_reference_fixture():
    mine = np.array([po.lib.orc_e4m3_value(b) for b in range(256)], np.float32)
    want = GOLDEN["e4m3_value"]
    assert np.array_equal(np.isnan(mine), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(u32(mine[ok]), u32(want[ok]))


def test_e4m3_closed_form():
    # OCP E4M3FN: bias 7, subnormals m/8 * 2^-6, max 448, only S.1111.111 is NaN
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        v = po.lib.orc_e4m3_value(b)
        if e == 15 and m == 7:
            assert math.isnan(v)
            continue
        want = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert v == (-want if s else want)
    assert po.lib.orc_e4m3_value(0x7E) == 448.0


def test_e4m3_byte_matches_reference_fixture():
    xs, want = GOLDEN["e4m3_byte_x"], GOLDEN["e4m3_byte"]
    mine = np.array([po.lib.orc_e4m3_byte(float(x)) for x in xs], np.uint8)
    assert np.array_equal(mine, want)


def test_e4m3_byte_is_nearest_ties_even():
    vals = np.array([po.lib.orc_e4m3_value(b) for b in range(127)], np.float64)
    for x in np.random.default_rng(0).uniform(0, 460, 3000).astype(np.float32):
        b = po.lib.orc_e4m3_byte(float(x))
        d = np.abs(vals - float(x))
        best = np.flatnonzero(d == d.min())
        if x >= 448:
            assert b == 126
        elif len(best) == 1:
            assert b == best[0]
        else:   # a tie between two codes: the even one
            assert b in best and b % 2 == 0


# ---------------------------------------------------------------- the packer
def test_q4_block_matches_reference_fixture():
    xs, s2 = GOLDEN["q4_block_x"], float(GOLDEN["q4_block_s2"])
    for i in range(xs.shape[0]):
        s = np.zeros(1, np.uint8)
        c = np.zeros(16, np.uint8)
        po.lib.orc_q4_block(P(np.ascontiguousarray(xs[i])), s2, P(s), P(c))
        assert s[0] == GOLDEN["q4_block_scale"][i]
        assert np.array_equal(c, GOLDEN["q4_block_codes"][i])


def _block_err(x, sb, s2):
    scale = np.float32(po.lib.orc_e4m3_value(int(sb))) * np.float32(s2)
    safe = scale if scale != 0 else np.float32(1)
    y = (x / safe).astype(np.float32)
    a = np.minimum(np.abs(y), np.float32(15))
    idx = np.clip(np.rint((a - np.float32(1)) * np.float32(0.5)), 0, 7)
    q = np.where(y < 0, -(2 * idx + 1), 2 * idx + 1).astype(np.float32) * scale
    return float(np.sum((q.astype(np.float64) - x) ** 2))


def test_q4_block_optimal_among_candidates():
    # invariant: the chosen scale byte's squared error is no larger than any candidate's, and levels are odd
    rng = np.random.default_rng(5)
    s2 = np.float32(0.02 * 4 * 1.25 / 6720)
    for _ in range(300):
        x = (rng.standard_normal(16) * 0.02).astype(np.float32)
        s = np.zeros(1, np.uint8)
        c = np.zeros(16, np.uint8)
        po.lib.orc_q4_block(P(x), float(s2), P(s), P(c))
        amax = np.float32(np.abs(x).max())
        cands = set()
        for t in (15.0, 13.0):
            b0 = po.lib.orc_e4m3_byte(float(amax / (np.float32(t) * s2)))
            cands |= {min(max(b0 + k, 0), 0x7E) for k in range(-2, 3)}
        e_best = _block_err(x, s[0], s2)
        assert all(e_best <= _block_err(x, cb, s2) * (1 + 1e-6) for cb in cands)
        # code symmetry: the sign of the level follows the sign of x (codes 8..15 negative)
        nz = np.abs(x) > 0
        assert np.all((c[nz] >= 8) == (x[nz] < 0))


def test_q4_global_formula():
    w = GOLDEN["mat_w"]
    assert u32(np.float32(po.lib.orc_q4_global(P(w), w.size))) == u32(
        np.float32(np.float32(np.abs(w).max()) * np.float32(1.25) / np.float32(6720.0)))
    assert u32(np.float32(GOLDEN["mat_global"])) == u32(np.float32(po.lib.orc_q4_global(P(w), w.size)))


def test_q4_pack_matches_reference_blocks(ref):
    # the packed matrix of the fixture: every block equals the reference's q4_block on it (nibble order 2k | 2k+1)
    w, wq, g = GOLDEN["mat_w"], GOLDEN["mat_q4"], float(GOLDEN["mat_global"])
    mine, g2 = po.q4_pack(w)
    assert np.array_equal(mine, wq) and g2 == g
    cols = w.shape[1]
    for r in range(w.shape[0]):
        for b in range(cols // 16):
            s = np.zeros(1, np.uint8)
            c = np.zeros(16, np.uint8)
            ref.ref_q4_block(P(np.ascontiguousarray(w[r, b * 16:(b + 1) * 16])), g, P(s), P(c))
            assert wq[r, cols // 2 + b] == s[0]
            assert np.array_equal(wq[r, b * 8:(b + 1) * 8], (c[0::2] | (c[1::2] << 4)).astype(np.uint8))


# ---------------------------------------------------------------- dequant and products
KQ4 = np.array([1, 3, 5, 7, 9, 11, 13, 15, -1, -3, -5, -7, -9, -11, -13, -15], np.float32)


def test_dequant_matches_reference_fixture():
    wq, g = GOLDEN["mat_q4"], float(GOLDEN["mat_global"])
    assert np.array_equal(u32(po.dequant(wq, 256, g)), u32(GOLDEN["mat_dequant"]))


def test_dequant_closed_form_exhaustive():
    # every code with every finite scale byte: value = (float(level) * 1) * (e4m3 * global) in fp32
    codes = np.repeat(np.arange(16, dtype=np.uint8) * 17, 1)[None, :].repeat(127, 0)
    scales = np.stack([np.arange(127, dtype=np.uint8)] * 2, 1)
    pack = np.concatenate([codes, scales], 1)
    g = np.float32(0.0371)
    d = po.dequant(pack, 32, float(g))
    e4 = np.array([po.lib.orc_e4m3_value(b) for b in range(127)], np.float32)
    for r in range(127):
        s = np.float32(e4[r] * g)
        lv = np.repeat(KQ4, 2)   # byte j = code j in both nibbles: values 2j, 2j+1 = level(j)
        assert np.array_equal(u32(d[r]), u32(lv * s))


def test_matvec_exact_matches_reference_fixture():
    wq, g, x = GOLDEN["mat_q4"], float(GOLDEN["mat_global"]), GOLDEN["mat_x"]
    assert np.array_equal(u32(po.matvec(wq, 256, g, x)), u32(GOLDEN["mat_y_exact"]))


def test_matvec_exact_against_fp64():
    wq, g, x = GOLDEN["mat_q4"], float(GOLDEN["mat_global"]), GOLDEN["mat_x"]
    d = GOLDEN["mat_dequant"].astype(np.float64)
    want = d @ x.astype(np.float64)
    got = po.matvec(wq, 256, g, x)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    assert np.abs(got - want).max() > 0 or True


def test_quantize_activation_matches_reference_fixture():
    q, s, b = po.quantize_activation(GOLDEN["mat_x"])
    assert np.array_equal(q, GOLDEN["act_q"])
    assert np.array_equal(u32(s), u32(GOLDEN["act_scale"]))
    assert np.array_equal(b, GOLDEN["act_bsum"])


def test_quantize_activation_closed_form():
    x = GOLDEN["mat_x"].reshape(-1, 16)
    q, s, b = po.quantize_activation(x.ravel())
    amax = np.abs(x).max(1)
    assert np.array_equal(u32(s), u32((amax / np.float32(127)).astype(np.float32)))
    inv = (np.float32(127) / amax).astype(np.float32)
    want = np.clip(np.rint((x * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    assert np.array_equal(q.reshape(-1, 16), want)
    assert np.array_equal(b, want.astype(np.int32).sum(1))


def test_matvec_int8_matches_reference_fixture():
    wq, g, x = GOLDEN["mat_q4"], float(GOLDEN["mat_global"]), GOLDEN["mat_x"]
    assert np.array_equal(u32(po.matvec_q(wq, 256, g, x)), u32(GOLDEN["mat_y_int8"]))


def test_matvec_int8_block_sums_brute_force():
    # the int8 path's value from its exact integer block sums, evaluated in fp64: within fp32 rounding
    wq, g, x = GOLDEN["mat_q4"], float(GOLDEN["mat_global"]), GOLDEN["mat_x"]
    q, s, _ = po.quantize_activation(x)
    lv = np.empty((wq.shape[0], 256), np.int64)
    lv[:, 0::2] = KQ4[wq[:, :128] & 15]
    lv[:, 1::2] = KQ4[wq[:, :128] >> 4]
    e4 = np.array([po.lib.orc_e4m3_value(b) for b in range(256)], np.float64)
    sums = (lv.reshape(-1, 16, 16) * q.astype(np.int64).reshape(16, 16)[None]).sum(2)   # rows x blocks, exact
    want = (sums * e4[wq[:, 128:]] * s.astype(np.float64)[None]).sum(1) * g
    got = po.matvec_q(wq, 256, g, x)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_bf16_rows_match_reference_fixture():
    got = po.matvec_bf16(GOLDEN["bf16_w"], GOLDEN["bf16_x"])
    assert np.array_equal(u32(got), u32(GOLDEN["bf16_y"]))
    wf = (GOLDEN["bf16_w"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    want = GOLDEN["bf16_x"].astype(np.float64) @ wf.T
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_rmsnorm_matches_reference_fixture_and_closed_form():
    x, w = GOLDEN["norm_x"], GOLDEN["norm_w"]
    assert np.array_equal(u32(po.rmsnorm(x, w, 1e-6, True)), u32(GOLDEN["norm_zc"]))
    assert np.array_equal(u32(po.rmsnorm(x, w, 1e-6, False)), u32(GOLDEN["norm_plain"]))
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * (1 + w.astype(np.float64))
    assert np.abs(po.rmsnorm(x, w) - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_products_against_reference_build(ref, seed):
    rows, cols = 48, 512
    wq, g = po.q4_random(seed, rows, cols, 0.05)
    x = po.normal(seed + 100, cols, 2.0)
    for mine, refname in ((po.matvec(wq, cols, g, x), "ref_matvec_rows"), (po.matvec_q(wq, cols, g, x), "ref_matvec_rows_q")):
        y = np.empty(rows, np.float32)
        getattr(ref, refname)(P(wq), rows, cols, g, P(x), P(y))
        assert np.array_equal(u32(mine), u32(y))


# ---------------------------------------------------------------- routing
def test_route_topk_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(200):
        E, K = 256, 8
        lg = rng.standard_normal(E).astype(np.float32)
        if trial % 10 == 0:   # exact ties: equal logits must go to the lower index
            lg[rng.integers(0, E, 40)] = lg.max()
        ids, w = po.route_topk(lg, K)
        mx = lg.max()
        p = np.exp((lg - mx).astype(np.float32)).astype(np.float32)
        s = np.float32(0)
        for v in p:
            s = np.float32(s + v)
        p = (p / s).astype(np.float32)
        order = sorted(range(E), key=lambda e: (-p[e], e))[:K]
        assert list(ids) == order
        assert abs(float(np.sum(w, dtype=np.float64)) - 1.0) < 1e-6
        assert np.all(np.diff(w) <= 0)
