"""Writes tests/golden/ref_vectors.npz: inputs and outputs of the reference's own functions, compiled from its sources
in this container (oracle/_ref/libgeode_ref.so: engine/src/kernels.cpp, sampler.cpp, yue2_q4.cpp).

The fixtures are data only (seeded inputs and the reference's outputs); the GPU box, which has no reference tree,
checks the oracle against them. Run from the repository root after `make -C oracle ref`:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402


def main():
    ref = po.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libgeode_ref.so is not built (make -C oracle ref)")
    P = po._ptr
    out = {}
    # E4M3: every byte
    out["e4m3_value"] = np.array([ref.ref_e4m3_value(b) for b in range(256)], np.float32)
    # e4m3_byte: the values, the midpoints, just around them, random floats, edges
    v = out["e4m3_value"][:127].astype(np.float64)
    mids = (v[:-1] + v[1:]) / 2
    pts = np.concatenate([v, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                          np.nextafter(mids.astype(np.float32), np.float32(1e9)),
                          np.random.default_rng(1).uniform(0, 500, 1500), [0.0, -1.0, 448.0, 449.0, 1e-12]])
    pts = pts.astype(np.float32)
    out["e4m3_byte_x"] = pts
    out["e4m3_byte"] = np.array([ref.ref_e4m3_byte(float(x)) for x in pts], np.uint8)
    # q4_block on seeded blocks at several magnitudes
    rng = np.random.default_rng(2)
    blocks = (rng.standard_normal((400, 16)) * np.repeat(rng.choice([1e-3, 0.02, 0.3, 2.0], 400)[:, None], 16, 1))
    blocks = blocks.astype(np.float32)
    blocks[:8] = 0.0
    blocks[8:16, :8] = 0.0
    s2 = np.float32(np.abs(blocks).max() * np.float32(1.25) / np.float32(6720.0))
    sb = np.zeros(400, np.uint8)
    codes = np.zeros((400, 16), np.uint8)
    for i in range(400):
        b = np.ascontiguousarray(blocks[i])
        s = np.zeros(1, np.uint8)
        c = np.zeros(16, np.uint8)
        ref.ref_q4_block(P(b), float(s2), P(s), P(c))
        sb[i], codes[i] = s[0], c
    out["q4_block_x"], out["q4_block_s2"], out["q4_block_scale"], out["q4_block_codes"] = blocks, s2, sb, codes
    # a packed matrix and its products
    rows, cols = 64, 256
    w = po.normal(3, rows * cols, 0.02).reshape(rows, cols)
    wq, g = po.q4_pack(w)   # the oracle's packer; checked against ref_q4_block below in the tests
    out["mat_w"], out["mat_q4"], out["mat_global"] = w, wq, np.float32(g)
    d = np.empty((rows, cols), np.float32)
    ref.ref_dequant_rows(P(wq), rows, cols, g, P(d))
    out["mat_dequant"] = d
    x = (po.normal(4, cols, 1.0) * np.linspace(0.05, 4, cols, dtype=np.float32)).astype(np.float32)
    out["mat_x"] = x
    y = np.empty(rows, np.float32)
    ref.ref_matvec_rows(P(wq), rows, cols, g, P(x), P(y))
    out["mat_y_exact"] = y.copy()
    ref.ref_matvec_rows_q(P(wq), rows, cols, g, P(x), P(y))
    out["mat_y_int8"] = y.copy()
    q = np.empty(cols, np.int8)
    sc = np.empty(cols // 16, np.float32)
    bs = np.empty(cols // 16, np.int32)
    ref.ref_quantize_activation(P(x), cols, P(q), P(sc), P(bs))
    out["act_q"], out["act_scale"], out["act_bsum"] = q, sc, bs
    # bf16 rows x 3 tokens
    wb = (po.normal(5, 32 * cols, 0.05).view(np.uint32) >> 16).astype(np.uint16).reshape(32, cols)
    xs = po.normal(6, 3 * cols, 1.0).reshape(3, cols)
    yb = np.empty((3, 32), np.float32)
    ref.ref_matvec_bf16_multi(P(wb), 32, cols, 3, P(xs), P(yb))
    out["bf16_w"], out["bf16_x"], out["bf16_y"] = wb, xs, yb
    # rmsnorm (zero-centred and plain)
    xn = po.normal(7, 2048, 1.5)
    wn = po.normal(8, 2048, 0.1)
    on = np.empty(2048, np.float32)
    ref.ref_rmsnorm(P(xn), P(wn), P(on), 2048, 1e-6, 1)
    out["norm_x"], out["norm_w"], out["norm_zc"] = xn, wn, on.copy()
    ref.ref_rmsnorm(P(xn), P(wn), P(on), 2048, 1e-6, 0)
    out["norm_plain"] = on.copy()
    # the Sampler's own stream (mt19937_64), several settings
    lg = po.normal(9, 3000, 3.0)
    out["sample_logits"] = lg
    settings = [(0.7, 0.95, 0, 42), (1.0, 0.8, 20, 7), (0.0, 1.0, 0, 1), (0.5, 1.0, 0, 99), (1.3, 0.5, 0, 5)]
    draws = []
    for (t, p, k, s) in settings:
        o = np.empty(64, np.int32)
        ref.ref_sample_seeded(P(lg), lg.size, t, p, k, s, 64, P(o))
        draws.append(o)
    out["sample_settings"] = np.array(settings, np.float64)
    out["sample_draws"] = np.stack(draws)
    # tile8 (the reference's expert layout of q4 packs): two matrices of pack rows, their tiled bytes, and row 37 of
    # the second read back by the reference's own quad_row
    for name, (rows, cols, seed) in (("tile8_a", (64, 128, 11)), ("tile8_b", (96, 192, 12))):
        wq, _ = po.q4_pack(po.normal(seed, rows * cols, 0.02).reshape(rows, cols))
        tiled = np.empty_like(wq)
        ref.ref_to_tile8(rows, cols, P(wq), P(tiled))
        out[name + "_rows"], out[name + "_tiled"] = wq, tiled
    back = np.empty(192 // 16 * 9, np.uint8)
    ref.ref_tile8_row(P(out["tile8_b_tiled"]), 96, 192, 37, P(back))
    out["tile8_b_row37"] = back
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
