"""Benchmark of the speculative-decoding verify step on one MI355X (the driver's contract: one JSON line).

Workload (the metric's config): the full 40-layer 35B-A3B-shape verify step, gated
attention (16 query heads, 2 KV heads, head_dim 256, RoPE theta 1e7) plus the MoE (256 experts, top-8 softmax
routing, 1 shared expert, ff 512), vocab 151,936, q4 weights seeded on the device (N(0, 0.02) through the RTN
packer), an fp16 KV cache of 8,192 context positions N(0, 1). A step verifies k = 4 chained drafts plus the last
token (M = 5 rows): every layer, the final norm and lm_head, logits left on the device, then the GPU's greedy
sample-and-match of the drafts on those logits (gv_accept_match, its result copied to the host) — a timed step is
both. The drafts are the target model's own greedy continuation, so all of them stand (5 tokens emitted a step):
`value` (tok/s) is the ceiling of acceptance; `verify_steps_per_s` (the verify alone) is the headline figure
independent of it. The draft tree (M = 17) is timed in the same run (`tree_m17`).

    python bench.py [--steps K] [--warmup W] [--tree] [--kv-int8] [--no-cpu]
    python bench.py --config c2|c3|c5      (the acceptance rules; one MoE block at M = 5 or 512)
    python bench.py --config real          (the real model's shape: 30 Gated DeltaNet + 10 attention layers)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

C4 = dict(hidden=2048, vocab=151936, n_layers=40, n_experts=256, top_k=8, moe_ff=512, shared_ff=512, n_heads=16,
          n_kv_heads=2, head_dim=256, rope_dim=64, rope_theta=1e7, eps=1e-6, max_ctx=8192 + 64, max_rows=17)
# the real model (Qwen3.6-35B-A3B, engine/src/gpu_check.cpp:277-281): 30 Gated DeltaNet layers (16 key heads, 32 value
# heads, 128-wide, conv of 4) and 10 gated-attention layers (every fourth), vocab 248,320, the int8 KV cache
REAL = dict(C4, vocab=248320, kv_int8=1, gdn_k_heads=16, gdn_v_heads=32, gdn_k_dim=128, gdn_v_dim=128, conv_kernel=4,
            gdn_layers=[0 if l % 4 == 3 else 1 for l in range(40)], mtp=1)
CTX = 8192
SEED = 20261201
PEAK_HBM = 8.0e12   # MI355X HBM3E, bytes/s
COPY_BYTES = 256 << 20
# HBM bytes a launch of the dominant kernel moves, from rocprofv3 FETCH_SIZE / WRITE_SIZE passes (KiB a dispatch)
# scaled by what the same counters read for a copy of known size (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000); the
# commands and figures are in profiles/moe_up_c4_m5_traffic.md
PROFILED_TRAFFIC = {("moe_up", 5): (22704.1 * 2.000 + 94.6 * 1.000) * 1024}
Q4_ROW = lambda cols: cols // 16 * 9   # noqa: E731  bytes of a q4 row (engine/src/kernels.cpp:900-902)


def tree_parents():
    """the draft tree of configs[3]: 16 nodes under the root, branching 4 then 3 (17 rows)"""
    parents, frontier = [-1], [0]
    for b in (4, 3):
        nxt = []
        for p in frontier:
            for _ in range(b):
                parents.append(p)
                nxt.append(len(parents) - 1)
        frontier = nxt
    return np.array(parents, np.int32)


def algorithmic_bytes(cls, c, M, uniq_per_layer, ctx):
    """bytes a launch of kernel class cls must move at least (weights and KV read once, activations ignored when
    small), per launch; uniq_per_layer: distinct routed experts of each layer counted from the run"""
    H, F, V = c["hidden"], c["moe_ff"], c["vocab"]
    nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
    L = c["n_layers"]
    gu, dn = 2 * F * Q4_ROW(H), H * Q4_ROW(F)
    if cls == "moe_up":
        return sum((u + 1) * gu for u in uniq_per_layer) / L
    if cls == "moe_down":
        return sum((u + 1) * dn for u in uniq_per_layer) / L
    if cls == "qkv":
        return (nh * 2 * hd + 2 * nkv * hd) * Q4_ROW(H)
    if cls == "o_proj":
        return H * Q4_ROW(nh * hd)
    if cls == "lm_head":
        return V * Q4_ROW(H)
    if cls == "attention":   # K and V of every position: fp16, or int8 and a float scale a row
        return 2 * nkv * (ctx + M) * (hd + 4 if c.get("kv_int8") else hd * 2)
    if cls == "router":
        return (c["n_experts"] + 1) * H * 2
    nk, nv, dk, dv = c.get("gdn_k_heads", 0), c.get("gdn_v_heads", 0), c.get("gdn_k_dim", 0), c.get("gdn_v_dim", 0)
    if cls == "gdn_core":   # the recurrent state read once, each row's state written to its slot
        return nv * dk * dv * 4 * (1 + M)
    if cls == "gdn_qkvz":
        return (2 * nk * dk + 2 * nv * dv) * Q4_ROW(H)
    if cls == "gdn_out":
        return H * Q4_ROW(nv * dv)
    if cls == "gdn_ab":
        return 2 * nv * H * 2
    return None


def step_bytes(c, M, uniq_per_layer, ctx):
    """algorithmic bytes of one whole verify step: per layer the q|k|v, o and router weights, the norm weights, the
    touched routed experts' and the shared expert's weights and the KV cache read; then the lm_head and the rows'
    embeddings"""
    tot = 0
    for u in uniq_per_layer:
        tot += algorithmic_bytes("qkv", c, M, [u], ctx) + algorithmic_bytes("o_proj", c, M, [u], ctx)
        tot += algorithmic_bytes("router", c, M, [u], ctx) + 2 * c["hidden"] * 4 + 2 * c["head_dim"] * 4
        tot += (u + 1) * (2 * c["moe_ff"] * Q4_ROW(c["hidden"]) + c["hidden"] * Q4_ROW(c["moe_ff"]))
        tot += algorithmic_bytes("attention", c, M, [u], ctx)
    tot += algorithmic_bytes("lm_head", c, M, [0], ctx) + M * c["hidden"] * 4
    return tot


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    return po


def cpu_baseline(M, threads, kv_int8=False, budget_s=30.0):
    """The oracle (the reference's CPU arithmetic restated, int8 path; g++ -O3 -march=x86-64-v3, rows split over
    `threads` in chunks of 16 as ThreadPool::parallel_for) on the host cores: whole 40-layer verify steps of the same
    workload (full shapes, ctx 8192, timing-only random q4 bytes, every layer its own weights: ~20 GB of host memory),
    the best of the steps that fit the time budget (at least one)."""
    po = _oracle()
    po.lib.orc_set_threads(threads)
    cfg = dict(C4, kv_int8=int(kv_int8))
    om = po.Model(cfg, seed=SEED, ctx=CTX, fast=True)
    toks = (np.arange(M) * 1000 + 7).astype(np.int32)
    times = []
    t_start = time.time()
    while not times or (time.time() - t_start + times[-1] < budget_s and len(times) < 3):
        om.position = CTX
        t0 = time.perf_counter()
        om.verify(toks)
        times.append(time.perf_counter() - t0)
    del om
    best = min(times)
    return {"value": M / best, "unit": "tok/s", "cores": threads, "kind": "port",
            "verify_steps_per_s": 1.0 / best,
            "sample": f"whole 40-layer verify steps at full shapes, M={M}, ctx {CTX}, int8 path, "
                      f"{'int8' if kv_int8 else 'fp16'} KV; best of {len(times)}: {best * 1e3:.0f} ms a step"}


def cpu_baseline_one_core(M, kv_int8=False):
    """one core: a bounded sample (one of the 40 layers plus the final norm and lm_head at full shapes, the step
    extrapolated as t_head + 40 x t_layer; a whole step on one core takes ~1.5 minutes)"""
    po = _oracle()
    po.lib.orc_set_threads(1)
    cfg = dict(C4, kv_int8=int(kv_int8), n_layers=1)
    om = po.Model(cfg, seed=SEED, ctx=CTX, fast=True)
    toks = (np.arange(M) * 1000 + 7).astype(np.int32)
    best = None
    for _ in range(2):
        om.position = CTX
        om.verify(toks)
        tl, th = om.last_times()
        est = th + C4["n_layers"] * tl
        best = est if best is None else min(best, est)
    return {"value": M / best, "unit": "tok/s", "cores": 1,
            "sample": f"1 of 40 layers + final norm + lm_head at full shapes, M={M}; step = t_head + 40 x t_layer = "
                      f"{best * 1e3:.0f} ms"}


def bench_moe_block(g, M, reps):
    """C3 (M = 5) / C5 (M = 512): one MoE block at the configs' shapes (256 experts + the shared one, hidden 2048,
    ff 512), rows fp16-valued N(0, 1), routed logits N(0, 1) given; device time of the block re-run on its staged
    inputs (gv_model_moe_replay), each run on the next of 3 layers of distinct weights: 3 x 257 expert blocks =
    1.36 GB, more than the 256 MB Infinity Cache holds, so that every run reads its experts from HBM"""
    cfg = dict(C4)
    cfg["n_layers"] = 3
    m = g.VerifyModel(cfg)
    m.randomize(SEED, 0.02, 0.0221, 0)
    rng = np.random.default_rng(SEED + M)
    h = rng.standard_normal((M, cfg["hidden"])).astype(np.float16).astype(np.float32)
    lg = rng.standard_normal((M, cfg["n_experts"])).astype(np.float32)
    out, ids, _ = m.moe(0, h, lg)
    touched = len(np.unique(ids))
    ms = m.moe_replay(reps)
    blk = 2 * cfg["moe_ff"] * Q4_ROW(cfg["hidden"]) + cfg["hidden"] * Q4_ROW(cfg["moe_ff"])   # 1,769,472 B
    byts = (touched + 1) * blk + (M * cfg["hidden"] * (2 + 4) if M > cfg["max_rows"] else 0)
    flops = 2.0 * 3 * cfg["hidden"] * cfg["moe_ff"] * M * (cfg["top_k"] + 1)
    m.close()
    return ms, touched, byts, flops


def bench_c1(g, reps=240, copies=48):
    """C1: the dense SwiGLU FFN 2048 -> 6144 -> 2048 (gate, up [6144 x 2048], down [2048 x 6144], weights N(0, 0.02)
    packed by the library's own packer on the device), x fp16 N(0, 1) [5 x 2048]; device time of gv_ffn_swiglu cycling
    through `copies` copies of the weights at distinct addresses (48 x 21.2 MB = 1.02 GB > the 256 MB Infinity
    Cache), hipEvents around `reps` back-to-back calls"""
    import ctypes as C
    H, F, M = 2048, 6144, 5
    rng = np.random.default_rng(SEED + 1)
    glob = g.DeviceBuffer(16)
    mats = []
    for i, (rows, cols) in enumerate(((F, H), (F, H), (H, F))):   # gate, up, down: packed once, copied
        w = g.DeviceBuffer.from_array(rng.normal(0.0, 0.02, (rows, cols)).astype(np.float32))
        pack = g.DeviceBuffer(rows * Q4_ROW(cols))
        g.check(g.lib.gv_q4_pack(w.ptr, rows, cols, pack.ptr, glob.ptr), "gv_q4_pack")
        gl = float(glob.download(np.float32, (1,))[0])
        w.free()
        mats.append((rows, cols, pack, gl))
    sets, bufs = [], []
    for _ in range(copies):
        one = []
        for rows, cols, pack, gl in mats:
            buf = g.DeviceBuffer(g.lib.gv_q4_device_bytes(rows, cols))
            d = g.GvQ4()
            g.check(g.lib.gv_q4_from_pack(pack.ptr, rows, cols, gl, buf.ptr, C.byref(d)), "gv_q4_from_pack")
            bufs.append(buf)
            one.append(d)
        sets.append(one)
    x = g.DeviceBuffer.from_array(rng.standard_normal((M, H)).astype(np.float16))
    y = g.DeviceBuffer(M * H * 4)
    ws = g.DeviceBuffer(g.lib.gv_ffn_workspace_bytes(H, F, M))

    def call(i):
        a, b, d = sets[i % copies]
        g.check(g.lib.gv_ffn_swiglu(C.byref(a), C.byref(b), C.byref(d), M, x.ptr, y.ptr, ws.ptr), "gv_ffn_swiglu")

    for i in range(copies):
        call(i)
    g.check(g.lib.gv_synchronize(), "sync")
    e0 = g.lib.gv_event_record()
    for i in range(reps):
        call(i)
    e1 = g.lib.gv_event_record()
    us = g.lib.gv_event_elapsed_ms(e0, e1) / reps * 1e3
    byts = 2 * F * Q4_ROW(H) + H * Q4_ROW(F) + M * H * 2 + M * H * 4   # 21,295,104 B (fp16 in, fp32 out)
    return us, byts


def bench_c2(g, trials):
    """C2: target logits [5 x V] ~ N(0, 3), draft [4 x V] = target rows 0..3 + N(0, 0.5), T 0.7, top-p 0.95; the
    textbook rule per trial (seeded uniforms), stochastic and greedy, and sample-and-match of the 5 rows; logits
    resident on the device, the time of each API call (device work and the result copy)"""
    import ctypes as C
    V, k = C4["vocab"], 4
    rng = np.random.default_rng(SEED)
    target = (rng.standard_normal((k + 1, V)) * 3).astype(np.float32)
    draft = (target[:k] + rng.standard_normal((k, V)) * 0.5).astype(np.float32)
    dt, dd = g.DeviceBuffer.from_array(target), g.DeviceBuffer.from_array(draft)
    out = np.empty(k + 1, np.int32)
    res = {}
    for name, greedy in (("textbook_stochastic", 0), ("textbook_greedy", 1)):
        times, emitted = [], []
        for t in range(trials):
            r = np.random.default_rng(SEED + t)
            ud, ua = r.random(k).astype(np.float32), r.random(k).astype(np.float32)
            t0 = time.perf_counter()
            n = g.lib.gv_accept_textbook(dt.ptr, dd.ptr, V, V, k, 0.7, 0.95, greedy, ud.ctypes.data_as(C.c_void_p),
                                         ua.ctypes.data_as(C.c_void_p), float(r.random()),
                                         out.ctypes.data_as(C.c_void_p))
            times.append(time.perf_counter() - t0)
            g.check(-1 if n < 0 else 0, "gv_accept_textbook")
            emitted.append(n)
        res[name] = {"us_per_trial": float(np.median(times[2:]) * 1e6), "mean_tokens": float(np.mean(emitted))}
    batch = np.array([7, 1, 2, 3, 4], np.int32)
    kept = C.c_int(0)
    times = []
    for t in range(trials):
        u = np.random.default_rng(SEED + 7 * t).random(k + 1)
        t0 = time.perf_counter()
        n = g.lib.gv_accept_match(dt.ptr, V, V, batch.ctypes.data_as(C.c_void_p), k + 1, 0.7, 0.95, 0, 1024,
                                  u.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p), C.byref(kept))
        times.append(time.perf_counter() - t0)
        g.check(-1 if n < 0 else 0, "gv_accept_match")
    res["sample_and_match"] = {"us_per_step": float(np.median(times[2:]) * 1e6)}
    return res


def calibrate_copy(args):
    """a device-to-device vector copy of COPY_BYTES, three times: a kernel whose HBM traffic is known (COPY_BYTES read
    and COPY_BYTES written per launch), for scaling the FETCH_SIZE / WRITE_SIZE counters of a profile"""
    import geode_amd as g

    g.init(0)
    src, dst = g.lib.gv_malloc(COPY_BYTES), g.lib.gv_malloc(COPY_BYTES)
    g.check(g.lib.gv_memset(src, 1, COPY_BYTES))
    g.check(g.lib.gv_synchronize())
    e0 = g.lib.gv_event_record()
    for _ in range(3):
        g.check(g.lib.gv_memcpy_d2d(dst, src, COPY_BYTES))
    e1 = g.lib.gv_event_record()
    ms = g.lib.gv_event_elapsed_ms(e0, e1) / 3
    g.lib.gv_free(src)
    g.lib.gv_free(dst)
    print(json.dumps({"copy_bytes": COPY_BYTES, "ms_per_copy": ms, "gbs": 2 * COPY_BYTES / ms / 1e6}))


def bench_real(g, args):
    """The real model's shape: 30 Gated DeltaNet + 10 gated-attention layers, vocab 248,320, int8 KV, ctx 8,192;
    the chain (M = 5) and the 16-node tree (M = 17): device time of the verify step (graph replays back to back),
    the kernel classes' times, and the delta rule's launch against its state traffic."""
    C = REAL
    m = g.VerifyModel(C)
    m.randomize(SEED, 0.02, 0.0221, CTX)
    g.check(g.lib.gv_synchronize())
    out = {}
    gdn = [l for l in range(C["n_layers"]) if C["gdn_layers"][l]]
    for M, parents in ((5, None), (17, tree_parents())):
        toks = np.array([(7 + 1000 * i) % C["vocab"] for i in range(M)], np.int32)

        def step():
            m.position = CTX
            m.verify(toks, parents, want_logits=False)

        for _ in range(3):
            step()
        e0 = g.lib.gv_event_record()
        for _ in range(args.steps):
            step()
        e1 = g.lib.gv_event_record()
        ms = g.lib.gv_event_elapsed_ms(e0, e1) / args.steps
        per_class = {}
        for cls, name in enumerate(g.KERNEL_CLASSES):
            m.time_kernel(cls)
            for _ in range(3):
                step()
            tms, n = m.kernel_time()
            if n:
                per_class[name] = round(tms / 3, 4)
        m.time_kernel(-1)
        step()
        core_s = m.replay(g.KERNEL_CLASSES.index("gdn_core"), gdn[0], reps=60) / 1e3
        core_b = algorithmic_bytes("gdn_core", C, M, [], CTX)
        out[f"m{M}"] = {"rows": M, "ms_per_verify": ms, "verify_steps_per_s": 1e3 / ms,
                        "kernel_ms_per_step": per_class,
                        "gdn_core": {"avg_launch_us": core_s * 1e6, "bytes_per_launch": core_b,
                                     "achieved_gbs": core_b / core_s / 1e9, "frac": core_b / core_s / PEAK_HBM}}
    out["mtp"] = bench_drafts(g, m, args)
    m.close()
    return out


def bench_drafts(g, m, args):
    """The MTP draft layer after a chain verify (wall clock of the synchronous calls, each returning its token): a
    draft from the verify's 5 rows, a chained draft, the generate loop's chain of 4 drafts (pmin 0: all four), over
    the whole vocabulary and over a 32,768-token draft head (an example size of draft_vocab.bin)"""
    toks = np.array([(7 + 1000 * i) % REAL["vocab"] for i in range(5)], np.int32)
    m.position = CTX
    m.verify(toks, want_logits=False)
    res = {}
    for name, ids in (("whole_vocab", None), ("draft_vocab_32768", np.arange(0, REAL["vocab"], 7)[:32768])):
        m.set_draft_vocab(ids)

        def timed(fn, reps=max(5, args.steps)):
            for _ in range(2):
                fn()
            t0 = time.perf_counter()
            for _ in range(reps):
                fn()
            return (time.perf_counter() - t0) / reps * 1e3

        d = m.draft(toks, CTX)[0]
        res[name] = {"ms_draft_5_rows": timed(lambda: m.draft(toks, CTX)),
                     "ms_draft_next": timed(lambda: m.draft_next(d, CTX + 5)),
                     "ms_chain_4_drafts": timed(lambda: m.draft_chain(toks, CTX, 5, 0.0))}
    m.set_draft_vocab(None)
    return res


def main_config(args):
    import geode_amd as g

    g.init(0)
    if args.config == "real":
        r = bench_real(g, args)
        print(json.dumps({"metric": "real-shape verify steps/s (30 GDN + 10 attention layers)",
                          "value": r["m5"]["verify_steps_per_s"], "unit": "verify-steps/s", "n_gpus": 1,
                          "steps": args.steps, "higher_is_better": True, "dtype": "int8", "data": "synthetic",
                          "config": {"workload": "Qwen3.6-35B-A3B shape: 30 Gated DeltaNet (16/32 heads of 128, "
                                                 "conv 4) + 10 gated-attention layers, 256 experts top-8 + shared, "
                                                 "vocab 248320, int8 KV, ctx 8192; chain M=5 and tree M=17"},
                          "detail": r}))
        return
    if args.config == "c1":
        us, byts = bench_c1(g)
        print(json.dumps({"metric": "C1 dense SwiGLU FFN: HBM GB/s vs peak", "value": byts / (us / 1e6) / 1e9,
                          "unit": "GB/s", "n_gpus": 1, "steps": 240, "warmup": 48, "us_per_call": us,
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
                          "data": "synthetic",
                          "config": {"workload": "C1: 2048 -> 6144 -> 2048 SwiGLU FFN, M=5, x fp16 N(0,1), weights "
                                                 "N(0,0.02) q4, 48 weight copies rotated (1.02 GB)"},
                          "bytes_per_call": byts,
                          "roofline": {"bound": "hbm", "achieved": byts / (us / 1e6) / 1e9, "peak": PEAK_HBM / 1e9,
                                       "unit": "GB/s", "frac": byts / (us / 1e6) / PEAK_HBM, "traffic": None}}))
        return
    if args.config in ("c3", "c5"):
        M = 5 if args.config == "c3" else 512
        ms, touched, byts, flops = bench_moe_block(g, M, 20 if M > 5 else 100)
        out = {"metric": f"{args.config.upper()} MoE block: HBM GB/s vs peak", "value": byts / (ms / 1e3) / 1e9,
               "unit": "GB/s", "n_gpus": 1, "steps": 20 if M > 5 else 100, "warmup": 1, "ms_per_step": ms,
               "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
               "config": {"workload": f"{args.config.upper()}: one MoE block, 256 experts + shared, hidden 2048, ff 512, "
                                      f"top-8, M={M}, routed logits N(0,1) given"},
               "experts_touched": touched, "bytes_per_block": byts, "tflops": flops / (ms / 1e3) / 1e12,
               "roofline": {"bound": "hbm", "achieved": byts / (ms / 1e3) / 1e9, "peak": PEAK_HBM / 1e9,
                            "unit": "GB/s", "frac": byts / (ms / 1e3) / PEAK_HBM, "traffic": None}}
    else:
        r = bench_c2(g, 40)
        out = {"metric": "C2 acceptance: microseconds per trial", "value": r["textbook_stochastic"]["us_per_trial"],
               "unit": "us/trial", "n_gpus": 1, "steps": 40, "warmup": 2, "higher_is_better": False,
               "scaling": "weak", "vs_baseline": None, "dtype": "f32/f64", "data": "synthetic",
               "config": {"workload": "C2: k=4, V=151936, T=0.7, top-p 0.95, textbook rule (stochastic), logits "
                                      "device-resident; per API call incl. the result copy"}, "detail": r,
               "bytes_per_trial": 9 * C4["vocab"] * 4}
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tree", action="store_true", help="verify the 17-row draft tree instead of the k=4 chain")
    ap.add_argument("--kv-int8", action="store_true",
                    help="the int8 KV cache (the reference's default cache) instead of the configs' fp16")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only a 256 MiB device copy, three times: the known traffic that scales HBM byte counters")
    ap.add_argument("--config", choices=["c4", "c1", "c2", "c3", "c5", "real"], default="c4",
                    help="c4 (default): the verify step; c1: the dense SwiGLU FFN; c2 / c3 / c5: the acceptance rules "
                         "/ one MoE block; real: the real model's shape with its Gated DeltaNet layers")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the verify step on one GPU only: the step of one sequence does not shard "
              "(independent sequences go one a GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args)
        return
    if args.config != "c4":
        main_config(args)
        return

    import geode_amd as g

    g.init(0)
    C = dict(C4, kv_int8=1) if args.kv_int8 else C4
    M = 17 if args.tree else 5
    parents = tree_parents() if args.tree else None
    m = g.VerifyModel(C)
    t0 = time.time()
    m.randomize(SEED, 0.02, 0.0221, CTX)
    g.check(g.lib.gv_synchronize())
    t_init = time.time() - t0

    # the drafts: the model's own greedy continuation of a token (each verified alone, then rolled back)
    toks = [7]
    m.position = CTX
    for i in range(M - 1):
        lg = m.verify(np.array([toks[-1]], np.int32))
        toks.append(int(np.argmax(lg[0])))
    toks = np.array(toks, np.int32)
    if args.tree:   # a tree's first child of each node follows the chain, the rest other tokens
        toks = np.array([(7 + 1000 * i) % C["vocab"] for i in range(M)], np.int32)

    def step():
        m.position = CTX
        m.verify(toks, parents, want_logits=False)

    import ctypes as ct
    acc_out, kept, u0 = np.empty(M, np.int32), ct.c_int(0), np.zeros(M)

    def step_accept():
        """the verify, then the GPU's greedy sample-and-match of the chain on its device logits (geode.cpp:318-374)"""
        step()
        n = g.lib.gv_accept_match(g.lib.gv_model_logits(m.h), C["vocab"], C["vocab"], toks.ctypes.data_as(ct.c_void_p),
                                  M, 0.0, 1.0, 0, 1024, u0.ctypes.data_as(ct.c_void_p),
                                  acc_out.ctypes.data_as(ct.c_void_p), ct.byref(kept))
        g.check(-1 if n < 0 else 0, "gv_accept_match")
        return n

    timed = step if args.tree else step_accept   # the tree's acceptance is a walk on the host, not timed
    for _ in range(args.warmup):
        timed()
    g.check(g.lib.gv_synchronize())
    t0 = time.perf_counter()
    e0 = g.lib.gv_event_record()
    for _ in range(args.steps):
        timed()
    e1 = g.lib.gv_event_record()
    g.check(g.lib.gv_synchronize())
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_events = g.lib.gv_event_elapsed_ms(e0, e1) / args.steps
    # the verify alone (graph replays back to back, no host wait between them)
    e0 = g.lib.gv_event_record()
    for _ in range(args.steps):
        step()
    e1 = g.lib.gv_event_record()
    ms_verify = g.lib.gv_event_elapsed_ms(e0, e1) / args.steps
    # the same steps as plain launches (no graph), for comparison
    m.set_graphs(False)
    e0 = g.lib.gv_event_record()
    for _ in range(args.steps):
        step()
    e1 = g.lib.gv_event_record()
    ms_direct = g.lib.gv_event_elapsed_ms(e0, e1) / args.steps
    m.set_graphs(True)

    # acceptance of the last step's logits: the GPU's own count for the chain (checked against the host's greedy
    # walk), a greedy walk on the host for the tree
    m.position = CTX
    logits = m.verify(toks, parents)
    route = m.route_ids(M)
    uniq = [len(np.unique(route[l])) for l in range(C["n_layers"])]
    if not args.tree:
        emitted = step_accept()
        host = 1
        for i in range(M - 1):
            if int(np.argmax(logits[i])) != int(toks[i + 1]):
                break
            host += 1
        assert host == emitted, f"GPU acceptance emitted {emitted} tokens, the host's greedy walk {host}"
    else:
        emitted = 1
        node = 0
        while True:
            y = int(np.argmax(logits[node]))
            kids = [j for j in range(M) if parents[j] == node and toks[j] == y]
            if not kids:
                break
            node = kids[0]
            emitted += 1

    # per kernel class: the summed event time over some timed steps (events around each launch: dispatch included)
    per_class = {}
    for cls, name in enumerate(g.KERNEL_CLASSES):
        m.time_kernel(cls)
        for _ in range(3):
            step()
        tms, n = m.kernel_time()
        per_class[name] = (tms / 3, n // 3)
    m.time_kernel(-1)
    # the dominant kernel: the class moving the most algorithmic bytes a step (the experts' gate|up products)
    dom = max((k for k in per_class if algorithmic_bytes(k, C, M, uniq, CTX)),
              key=lambda k: algorithmic_bytes(k, C, M, uniq, CTX) * max(per_class[k][1], 1))
    # the dominant kernel's launch time: its launches of every layer replayed back to back between two events on
    # the step's own state, each launch on the next layer's weights (none of them cached by the previous launch)
    m.position = CTX
    m.verify(toks, parents, want_logits=False)
    cls = g.KERNEL_CLASSES.index(dom)
    dom_avg_s = m.replay(cls, 0, reps=2 * C["n_layers"]) / 1e3
    dom_bytes = algorithmic_bytes(dom, C, M, uniq, CTX)
    achieved = dom_bytes / dom_avg_s

    steps_s = 1e3 / ms
    verify_steps_s = 1e3 / ms_verify
    sbytes = step_bytes(C, M, uniq, CTX)
    tree = None
    if not args.tree:   # the draft tree of configs[3] on the same model: 16 nodes (4, 3) + the root, M = 17
        tp = tree_parents()
        ttoks = np.array([(7 + 1000 * i) % C["vocab"] for i in range(17)], np.int32)

        def tstep():
            m.position = CTX
            m.verify(ttoks, tp, want_logits=False)

        for _ in range(3):
            tstep()
        e0 = g.lib.gv_event_record()
        for _ in range(args.steps):
            tstep()
        e1 = g.lib.gv_event_record()
        tms = g.lib.gv_event_elapsed_ms(e0, e1) / args.steps
        m.position = CTX
        m.verify(ttoks, tp, want_logits=False)
        troute = m.route_ids(17)
        tuniq = [len(np.unique(troute[l])) for l in range(C["n_layers"])]
        tbytes = step_bytes(C, 17, tuniq, CTX)
        tree = {"rows": 17, "ms_per_step": tms, "verify_steps_per_s": 1e3 / tms, "verified_rows_per_s": 17e3 / tms,
                "step_bytes": tbytes, "step_roofline_frac": tbytes / (tms / 1e3) / PEAK_HBM,
                "distinct_experts_per_layer": float(np.mean(tuniq))}
    out = {
        "metric": "verify-step tok/s, 35B-A3B-shape MoE k=4; HBM GB/s vs peak",
        "value": steps_s * emitted,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": ("C4 full 40-layer 35B-A3B-shape verify step, " +
                                ("draft tree 16 nodes (4,3) + root, M=17" if args.tree else "chain k=4, M=5") +
                                f", ctx {CTX}, vocab 151936, q4 weights, {'int8' if args.kv_int8 else 'fp16'} KV, int8-path products"),
                   "rows": M, "tokens_emitted_per_step": emitted, "acceptance": "greedy sample-and-match on the "
                   "step's logits; drafts = the target's own greedy chain" if not args.tree else "greedy tree walk"},
        "value_note": "tok/s with every draft accepted (the drafts are the target's own greedy chain): the ceiling "
                      "of acceptance; verify_steps_per_s is the step rate that does not depend on it",
        "verify_steps_per_s": verify_steps_s,
        "ms_per_verify": ms_verify,
        "ms_per_step_device_events": ms_events,
        "ms_per_verify_without_graphs": ms_direct,
        "verified_rows_per_s": verify_steps_s * M,
        "step_hbm_gbs": sbytes / (ms_verify / 1e3) / 1e9,
        "step_roofline_frac": sbytes / (ms_verify / 1e3) / PEAK_HBM,
        "step_bytes": sbytes,
        "distinct_experts_per_layer": float(np.mean(uniq)),
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM, "traffic": PROFILED_TRAFFIC.get((dom, M)),
                     "bytes_per_launch": dom_bytes, "avg_launch_us": dom_avg_s * 1e6,
                     "timing": "hipEvents around 80 back-to-back launches cycling through the 40 layers "
                               "(gv_model_replay)"},
        "kernel_ms_per_step": {k: round(v[0], 4) for k, v in per_class.items() if v[1]},
        "init_s": t_init,
    }
    if tree:
        out["tree_m17"] = tree
    if not args.no_cpu:
        # the host's threads as the process may use them, within the box's CPU share for one GPU (16 threads,
        # whatever os.cpu_count() shows there); and one core
        host = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        threads = min(16, host)
        out["cpu_baseline"] = cpu_baseline(M, threads, args.kv_int8)
        out["cpu_baseline"]["host_threads"] = os.cpu_count()
        out["cpu_baseline"]["one_core"] = cpu_baseline_one_core(M, args.kv_int8)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
