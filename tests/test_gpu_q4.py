"""GPU parity of the q4 path (C ABI) against the oracle: dequant and the packer bit for bit, the int8 activation codes
bit for bit, the skinny products (matrix cores) within fp32 summation order of the int8 path, the C1 dense SwiGLU
MLP within 1e-2."""
import numpy as np
import pytest

import pyoracle as po

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gv():
    import geode_amd

    geode_amd.init(0)
    return geode_amd


def _u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("rows,cols", [(64, 128), (300, 256), (256, 512), (1024, 2048), (520, 6144)])
def test_dequant_bit_exact(gv, rows, cols):
    wq, s2 = po.q4_random(11 + rows, rows, cols)
    m = gv.Q4Matrix(wq, rows, cols, s2)
    got = m.dequant()
    want = po.dequant(wq, cols, s2)
    assert np.array_equal(_u32(got), _u32(want))


def test_dequant_every_code_and_scale(gv):
    # every code byte with every finite scale byte: rows of 128 values, 8 blocks, scales 0..0x7E
    rows, cols = 127, 128
    codes = np.tile(np.arange(16, dtype=np.uint8) * 17, 4)[None, :].repeat(rows, 0)  # both nibbles equal
    sc = np.arange(127, dtype=np.uint8)
    scales = np.stack([sc, sc[::-1], (sc + 7) % 127, (sc + 50) % 127, sc, sc[::-1], (sc * 3) % 127, (sc + 99) % 127], 1)
    pack = np.concatenate([codes, scales], 1)
    m = gv.Q4Matrix(pack, rows, cols, 0.37)
    assert np.array_equal(_u32(m.dequant()), _u32(po.dequant(pack, cols, 0.37)))


@pytest.mark.parametrize("rows,cols", [(64, 256), (1000, 2048)])
def test_packer_bit_exact(gv, rows, cols):
    w = po.normal(21 + rows, rows * cols, 0.02).reshape(rows, cols)
    dw = gv.DeviceBuffer.from_array(w)
    out = gv.DeviceBuffer(rows * cols // 16 * 9)
    g = gv.DeviceBuffer(4)
    gv.check(gv.lib.gv_q4_pack(dw.ptr, rows, cols, out.ptr, g.ptr), "pack")
    got = out.download(np.uint8, (rows, cols // 16 * 9))
    s2 = g.download(np.float32, (1,))[0]
    want, s2w = po.q4_pack(w)
    assert _u32(np.float32(s2)) == _u32(np.float32(s2w))
    assert np.array_equal(got, want)


def _act16_values(raw, cols):
    """the products' operands (per 32-value chunk and 8-value group: 8 hi then 8 lo halves, values in the order
    0 4 1 5 2 6 3 7) back to one fp64 value per column"""
    h = raw.reshape(cols // 32, 4, 2, 8).astype(np.float64)
    v = h[:, :, 0, :] + h[:, :, 1, :]
    order = [0, 4, 1, 5, 2, 6, 3, 7]
    out = np.empty((cols // 32, 4, 8))
    for slot, u in enumerate(order):
        out[:, :, u] = v[:, :, slot]
    return out.reshape(cols)


@pytest.mark.parametrize("norm", [False, True])
def test_quantize_bit_exact(gv, norm):
    M, cols = 5, 2048
    x = po.normal(5, M * cols, 1.0).reshape(M, cols) * np.linspace(0.1, 3, cols, dtype=np.float32)
    w = po.normal(6, cols, 0.02)
    dx = gv.DeviceBuffer.from_array(x)
    dw = gv.DeviceBuffer.from_array(w)
    act = gv.DeviceBuffer(M * gv.act_bytes(cols))
    h = gv.DeviceBuffer(M * cols * 4)
    gv.check(gv.lib.gv_quantize(dx.ptr, cols, M, cols, dw.ptr if norm else None, 1e-6, act.ptr, h.ptr), "quantize")
    raw = act.download(np.float16, (M, cols * 2))
    hh = h.download(np.float32, (M, cols))
    for t in range(M):
        xt = po.rmsnorm(x[t], w) if norm else x[t]
        assert np.array_equal(_u32(hh[t]), _u32(xt))          # the RMSNorm bit for bit
        q, s, _ = po.quantize_activation(xt)
        val = _act16_values(raw[t], cols)
        srep = np.repeat(s.astype(np.float64), 16)
        assert np.array_equal(np.rint(val / np.where(srep > 0, srep, 1)).astype(np.int64), q)   # the int8 codes
        want = (q.astype(np.float32) * np.repeat(s, 16)).astype(np.float64)                   # q x scale in fp32
        assert np.abs(val - want).max() <= 2.0 ** -21 * np.abs(want).max()                    # as hi + lo halves


@pytest.mark.parametrize("rows,cols,M", [(64, 128, 1), (256, 256, 3), (1024, 2048, 5), (2048, 512, 5),
                                          (2048, 4096, 17), (9216, 2048, 5), (600, 2048, 32), (8192, 6144, 16)])
def test_gemv_int8_path(gv, rows, cols, M):
    wq, s2 = po.q4_random(31 + rows + cols, rows, cols)
    m = gv.Q4Matrix(wq, rows, cols, s2)
    x = po.normal(41 + M, M * cols, 1.0).reshape(M, cols)
    got = gv.gemv(m, x)
    want = np.stack([po.matvec_q(wq, cols, s2, x[t]) for t in range(M)])
    exact = np.stack([po.matvec(wq, cols, s2, x[t]) for t in range(M)])
    scale = np.abs(exact).max()
    # the integer block sums are exact; only the fp32 sum over blocks is in another order
    assert np.abs(got - want).max() <= 1e-5 * scale
    # and the gpu_check.cpp:80-94 criterion against the exact path
    err_gpu = np.abs(got - exact).max()
    err_int8 = np.abs(want - exact).max()
    assert err_gpu <= 1.5 * err_int8 + 1e-6 * scale


def test_gemv_accumulate(gv):
    rows, cols, M = 512, 2048, 4
    wq, s2 = po.q4_random(77, rows, cols)
    m = gv.Q4Matrix(wq, rows, cols, s2)
    x = po.normal(78, M * cols).reshape(M, cols)
    base = po.normal(79, M * rows).reshape(M, rows)
    got = gv.gemv(m, x, accumulate_into=base)
    want = base + np.stack([po.matvec_q(wq, cols, s2, x[t]) for t in range(M)])
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("M", [5, 8, 9, 17])
def test_c1_ffn_swiglu(gv, M):
    """C1: hidden 2048 -> 6144 -> 2048 SwiGLU, weights N(0, 0.02) packed, x fp16 N(0,1) at M = 5 (and 8: the fused
    three-launch path; 9, 17: the general one)."""
    H, F = 2048, 6144
    gq, gg = po.q4_random(1001, F, H)
    uq, ug = po.q4_random(1002, F, H)
    dq, dg = po.q4_random(1003, H, F)
    x16 = po.f32_to_f16_bits(po.normal(2001, M * H).reshape(M, H))
    G, U, D = gv.Q4Matrix(gq, F, H, gg), gv.Q4Matrix(uq, F, H, ug), gv.Q4Matrix(dq, H, F, dg)
    dx = gv.DeviceBuffer.from_array(x16)
    y = gv.DeviceBuffer(M * H * 4)
    ws = gv.DeviceBuffer(gv.lib.gv_ffn_workspace_bytes(H, F, M))
    gv.check(gv.lib.gv_ffn_swiglu(G.ref(), U.ref(), D.ref(), M, dx.ptr, y.ptr, ws.ptr), "ffn")
    got = y.download(np.float32, (M, H))
    want = po.ffn_swiglu(gq, uq, dq, gg, ug, dg, H, F, x16, mode=0)
    exact = po.ffn_swiglu(gq, uq, dq, gg, ug, dg, H, F, x16, mode=1)
    scale = np.abs(exact).max()
    # parity with the reference's default (int8) CPU path: max error within 1e-2 of the output's scale
    assert np.abs(got - want).max() <= 1e-2 * scale
    assert np.sqrt(np.mean((got - want) ** 2)) <= 1e-3 * np.sqrt(np.mean(want ** 2))
    # and the gpu_check.cpp:80-94 criterion against the exact path
    assert np.abs(got - exact).max() <= 1.5 * np.abs(want - exact).max() + 1e-6 * scale
