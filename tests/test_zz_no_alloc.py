"""gv_ffn_swiglu_noalloc (no reference counterpart: the C1 dense SwiGLU FFN for callers that cannot allocate) through
the C ABI against gv_ffn_swiglu with a caller's workspace, bit for bit: the same kernels on a different workspace.
Two calls in a row, the second with fewer rows (the scratch keeps the first call's contents); a shape whose workspace
exceeds the scratch is refused before any work."""
import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def test_noalloc_matches_workspace_entry_point(gv):
    H, F = 2048, 6144
    gq, gg = po.q4_random(1101, F, H)
    uq, ug = po.q4_random(1102, F, H)
    dq, dg = po.q4_random(1103, H, F)
    G, U, D = gv.Q4Matrix(gq, F, H, gg), gv.Q4Matrix(uq, F, H, ug), gv.Q4Matrix(dq, H, F, dg)
    for M, seed in ((17, 2101), (5, 2102)):   # the second call smaller than the first
        x16 = po.f32_to_f16_bits(po.normal(seed, M * H).reshape(M, H))
        dx = gv.DeviceBuffer.from_array(x16)
        y_ws, y_na = gv.DeviceBuffer(M * H * 4), gv.DeviceBuffer(M * H * 4)
        ws = gv.DeviceBuffer(gv.lib.gv_ffn_workspace_bytes(H, F, M))
        gv.check(gv.lib.gv_ffn_swiglu(G.ref(), U.ref(), D.ref(), M, dx.ptr, y_ws.ptr, ws.ptr), "gv_ffn_swiglu")
        gv.check(gv.lib.gv_ffn_swiglu_noalloc(G.ref(), U.ref(), D.ref(), M, dx.ptr, y_na.ptr), "noalloc")
        a = y_ws.download(np.float32, (M, H))
        b = y_na.download(np.float32, (M, H))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"M {M}: results differ"
        want = po.ffn_swiglu(gq, uq, dq, gg, ug, dg, H, F, x16, mode=0)
        assert np.abs(b - want).max() <= 1e-2 * np.abs(want).max()


def test_noalloc_refuses_a_shape_past_its_scratch(gv):
    H, F, M = 2048, 16384, 32   # a workspace of about 8.5 MB
    assert gv.lib.gv_ffn_workspace_bytes(H, F, M) > 4 << 20
    gq, gg = po.q4_random(1201, 128, H)   # (descriptors of the right shape are enough: the call is refused first)
    G = gv.Q4Matrix(gq, 128, H, gg)
    desc = gv.GvQ4(G.desc.codes, G.desc.scales, F, H, 0, 0, gg)
    ddesc = gv.GvQ4(G.desc.codes, G.desc.scales, H, F, 0, 0, gg)
    rc = gv.lib.gv_ffn_swiglu_noalloc(desc, desc, ddesc, M, G.buf.ptr, G.buf.ptr)
    assert rc != 0 and "scratch" in gv.lib.gv_last_error().decode()
