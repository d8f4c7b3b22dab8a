"""GPU parity at BASELINE.json configs[0] (C1, the dense SwiGLU FFN through the NPU plugin's calls) and configs[4]
(C5, the prefill-sized MoE chunk) at their own shapes, and the NPU plugin's other calls (gv_open / gv_adopt_q4 /
gv_gemm / gv_mlp, the C ABI of npu/host/npu_api.h:16-66) against the oracle's int8 path.

C5: hidden 2048, 256 experts + 1 shared of ff 512, top-8, M = 512 rows of fp16-valued N(0, 1), router logits N(0, 1)
given; the expert-grouped products (runs of at most 32 rows an expert) then the weighted combine, against
po.moe_layer: routed ids identical, weights within 1e-6, the block's output within 1e-2 (max error over max |value|).
"""
import ctypes

import numpy as np
import pytest

import pyoracle as po
from model_helpers import rel_err

pytestmark = pytest.mark.gpu

C5 = dict(hidden=2048, vocab=1024, n_layers=1, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
          n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=128, max_rows=17)


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def _f16_valued(seed, n):
    x = po.normal(seed, n, 1.0)
    return x.astype(np.float16).astype(np.float32)


def test_c5_prefill_moe_at_its_shape(gv):
    from model_helpers import adopt_oracle_model

    om = po.Model(C5, seed=41, router_sigma=1.0 / np.sqrt(C5["hidden"]), ctx=0, fast=True)
    gm = gv.VerifyModel(C5)
    try:
        adopt_oracle_model(gm, om, 0)
        M, H, E = 512, C5["hidden"], C5["n_experts"]
        h = _f16_valued(42, M * H).reshape(M, H)
        lg = po.normal(43, M * E, 1.0).reshape(M, E)
        want, wids, wwts = po.moe_layer(om, 0, h, lg)
        got, gids, gwts = gm.moe(0, h, lg)
        touched = len(np.unique(wids))
        err = rel_err(got, want)
        print(f"C5 M {M}: {touched} experts touched, max error {err:.3e}", flush=True)
        assert np.array_equal(gids, wids)
        assert np.abs(gwts - wwts).max() <= 1e-6
        assert err <= 1e-2
    finally:
        gm.close()


@pytest.mark.parametrize("shape", [dict(), dict(n_experts=100, top_k=6), dict(exact=1)],
                         ids=["e256k8", "e100k6", "exact"])
@pytest.mark.parametrize("M", [5, 8, 18, 37, 512, 1000])
def test_c5_fused_front_matches_the_separate_launches(gv, shape, M):
    """the MoE block's launches before the experts' products (prefill.hip) against the separate ones
    (gv_model_set_fused(m, 0)): the block's output, routed ids and weights bit for bit, in both arithmetic modes (the
    exact path's operands are the fp32 rows). Past the decode path's rows (max_rows 17), up to 1,000 (a ragged last
    group of four rows; two batches of picks to place): the routes, then the grouping with the shared expert's gate
    and the operands, against five launches; at 5 and 8 rows: the gate and operand roles against the router launch."""
    cfg = dict(C5, **shape)
    gm = gv.VerifyModel(cfg)
    try:
        gm.randomize(44, 0.02, 0.0221, 0)
        h = _f16_valued(45 + M, M * cfg["hidden"]).reshape(M, cfg["hidden"])
        lg = po.normal(46 + M, M * cfg["n_experts"], 1.0).reshape(M, cfg["n_experts"])
        fused = gm.moe(0, h, lg)
        gm.set_fused(0)
        apart = gm.moe(0, h, lg)
        for a, b in zip(fused, apart):   # (output, ids, weights)
            assert a.dtype == b.dtype and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        gm.close()


# ---------------------------------------------------------------- the NPU plugin's calls
def _open(gv):
    lib = gv.lib
    err = ctypes.create_string_buffer(256)
    h = lib.gv_open(0, err, 256)
    assert h, err.value
    return lib, h


def _adopt(lib, h, wq, rows, cols, g):
    wq = np.ascontiguousarray(wq, np.uint8)
    i = lib.gv_adopt_q4(h, wq.ctypes.data_as(ctypes.c_void_p), rows, cols, cols // 16 * 9, g)
    assert i >= 0, gv_err(lib)
    return i


def gv_err(lib):
    return lib.gv_last_error().decode()


def _rowptrs(a):
    return (ctypes.c_void_p * a.shape[0])(*[a[i].ctypes.data for i in range(a.shape[0])])


@pytest.mark.parametrize("rows,cols,n", [(256, 512, 1), (1024, 2048, 5), (520, 6144, 37), (2048, 4096, 17),
                                         (256, 4096, 32), (9216, 2048, 17), (9000, 2048, 25)])
def test_npu_gemm(gv, rows, cols, n):
    """gnpu_gemm's contract (npu_api.h:42-44): ys[t] = W xs[t], fp32 rows in and out; n past 32 rows in batches;
    17..32 rows over K = 4096 (the rows in two groups of one launch) and over K = 2048 (a ragged last tile)"""
    lib, h = _open(gv)
    try:
        wq, g = po.q4_random(50 + rows, rows, cols, 0.02)
        i = _adopt(lib, h, wq, rows, cols, g)
        x = po.normal(60 + n, n * cols, 1.0).reshape(n, cols)
        y = np.zeros((n, rows), np.float32)
        assert lib.gv_gemm(h, i, n, _rowptrs(x), _rowptrs(y)) == 0, gv_err(lib)
        want = np.array([po.matvec_q(wq, cols, g, x[t]) for t in range(n)])
        assert rel_err(y, want) <= 1e-5
    finally:
        lib.gv_close(h)


def test_npu_mlp_c1_shape(gv):
    """gnpu_mlp's contract (npu_api.h:58-66) at C1's shape (2048 -> 6144 -> 2048, SwiGLU): ys[t] = down(silu(gate
    xs[t]) * up xs[t]), down adopted in two parts of its inputs whose results add; against the oracle's dense MLP"""
    lib, h = _open(gv)
    try:
        H, F, M = 2048, 6144, 5
        gq, gg = po.q4_random(71, F, H)
        uq, gu = po.q4_random(72, F, H)
        dq, gd = po.q4_random(73, H, F)
        ig = _adopt(lib, h, gq, F, H, gg)
        iu = _adopt(lib, h, uq, F, H, gu)
        # down in two parts of its columns (3072 each): the pack rows of each part, the same global
        half = F // 2
        parts = []
        for p in range(2):
            codes = dq[:, p * half // 2:(p + 1) * half // 2]
            scales = dq[:, F // 2 + p * half // 16:F // 2 + (p + 1) * half // 16]
            parts.append(_adopt(lib, h, np.concatenate([codes, scales], axis=1), H, half, gd))
        x16 = _f16_valued(74, M * H).reshape(M, H)
        y = np.zeros((M, H), np.float32)
        downs = (ctypes.c_int * 2)(*parts)
        assert lib.gv_mlp(h, ig, iu, 2, downs, 1, M, _rowptrs(x16), _rowptrs(y)) == 0, gv_err(lib)
        want = po.ffn_swiglu(gq, uq, dq, gg, gu, gd, H, F, po.f32_to_f16_bits(x16))
        err = rel_err(y, want)
        print(f"C1 via gv_mlp (down in two parts): max error {err:.3e}", flush=True)
        assert err <= 1e-2
        # the same with down whole
        idn = _adopt(lib, h, dq, H, F, gd)
        y1 = np.zeros((M, H), np.float32)
        assert lib.gv_mlp(h, ig, iu, 1, (ctypes.c_int * 1)(idn), 1, M, _rowptrs(x16), _rowptrs(y1)) == 0
        assert rel_err(y1, want) <= 1e-2
        # act 0 (gelu) is not served: an error, no partial work
        assert lib.gv_mlp(h, ig, iu, 1, (ctypes.c_int * 1)(idn), 0, M, _rowptrs(x16), _rowptrs(y1)) != 0
    finally:
        lib.gv_close(h)
