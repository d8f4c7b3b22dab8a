"""Shared by the model tests: small model shapes, the oracle model's tensors adopted by the GPU model, draft trees."""
import numpy as np

import pyoracle as po

# a small model of the C4 family (gated attention + MoE), quick for the oracle
SMALL = dict(hidden=256, vocab=512, n_layers=2, n_experts=16, top_k=4, moe_ff=128, shared_ff=128, n_heads=4,
             n_kv_heads=2, head_dim=64, rope_dim=16, rope_theta=1e7, eps=1e-6, max_ctx=160, max_rows=17)
# router sigma giving unit-std router logits for unit-RMS inputs
SMALL_ROUTER_SIGMA = 1.0 / np.sqrt(SMALL["hidden"])


def tree_parents(branching=(4, 3)):
    """BFS parents of a draft tree under a root: 1 root, then each depth's nodes with `branching[d]` children each."""
    parents = [-1]
    frontier = [0]
    for b in branching:
        nxt = []
        for p in frontier:
            for _ in range(b):
                parents.append(p)
                nxt.append(len(parents) - 1)
        frontier = nxt
    return np.array(parents, np.int32)


def adopt_oracle_model(gm, om, ctx):
    """Copy every tensor of the oracle model (pack layout) into the GPU model."""
    import geode_amd as g

    c = om.cfg
    H, F, hd, nkv = c["hidden"], c["moe_ff"], c["head_dim"], c["n_kv_heads"]
    t, gl = om.tensor(po.EMBED)
    gm.adopt(g.EMBED, t, globals_=gl[:1])
    t, gl = om.tensor(po.LM_HEAD)
    gm.adopt(g.LM_HEAD, t, globals_=gl[:1])
    gm.adopt(g.FINAL_NORM, om.tensor(po.FINAL_NORM)[0])
    gdn = c.get("gdn_layers", ())
    if c.get("mtp"):   # the MTP layer's own tensors; its decoder layer is layer n_layers below
        t, gl = om.tensor(po.MTP_FC)
        gm.adopt(g.MTP_FC, t, globals_=gl[:1])
        for k_o, k_g in ((po.MTP_NORM, g.MTP_NORM), (po.MTP_PRE_E, g.MTP_PRE_E), (po.MTP_PRE_H, g.MTP_PRE_H)):
            gm.adopt(k_g, om.tensor(k_o)[0])
    for l in range(c["n_layers"] + (1 if c.get("mtp") else 0)):
        for k_o, k_g in ((po.IN_NORM, g.IN_NORM), (po.POST_NORM, g.POST_NORM), (po.ROUTER, g.ROUTER),
                         (po.SHARED_GATE, g.SHARED_GATE)):
            gm.adopt(k_g, om.tensor(k_o, l)[0], layer=l)
        if l < len(gdn) and gdn[l]:   # a Gated DeltaNet layer: its tensors, its states
            for k_o, k_g in ((po.GDN_QKV, g.GDN_QKV), (po.GDN_Z, g.GDN_Z), (po.GDN_OUT, g.GDN_OUT)):
                t, gl = om.tensor(k_o, l)
                gm.adopt(k_g, t, layer=l, globals_=gl[:1])
            for k_o, k_g in ((po.GDN_A, g.GDN_A), (po.GDN_B, g.GDN_B), (po.GDN_ALOG, g.GDN_ALOG),
                             (po.GDN_DTB, g.GDN_DTB), (po.GDN_CONV, g.GDN_CONV), (po.GDN_NORM, g.GDN_NORM),
                             (po.GDN_CONV_ST, g.GDN_CONV_ST), (po.GDN_S, g.GDN_S)):
                gm.adopt(k_g, om.tensor(k_o, l)[0], layer=l)
        else:
            for k_o, k_g in ((po.Q_NORM, g.Q_NORM), (po.K_NORM, g.K_NORM)):
                gm.adopt(k_g, om.tensor(k_o, l)[0], layer=l)
            q, gq = om.tensor(po.Q, l)
            k, gk = om.tensor(po.K, l)
            v, gv = om.tensor(po.V, l)
            gm.adopt(g.QKV, np.concatenate([q, k, v]), layer=l, globals_=[gq[0], gk[0], gv[0]])
            o, go = om.tensor(po.O, l)
            gm.adopt(g.O, o, layer=l, globals_=go[:1])
        for e in range(c["n_experts"]):
            blk, ge = om.tensor(po.EXPERT, l, e)
            gm.adopt(g.EXPERT, blk, layer=l, expert=e, globals_=ge)
        sg, gsg = om.tensor(po.SH_GATE, l)
        su, gsu = om.tensor(po.SH_UP, l)
        sd, gsd = om.tensor(po.SH_DOWN, l)
        gm.adopt(g.SHARED_EXPERT, np.concatenate([sg, su, sd]), layer=l, globals_=[gsg[0], gsu[0], gsd[0]])
        if l < len(gdn) and gdn[l]:
            continue
        if c.get("kv_int8"):   # the int8 rows and their scales, the reference's int8 chunk layout
            q, _ = om.tensor(po.KV8, l)
            sc, _ = om.tensor(po.KVS, l)
            q = q.reshape(2, c["max_ctx"], nkv * hd)[:, :ctx]
            sc = sc.view(np.float32).reshape(2, c["max_ctx"], nkv)[:, :ctx]
            gm.adopt(g.KV_I8, np.concatenate([q.reshape(-1), np.ascontiguousarray(sc).view(np.uint8).reshape(-1)]),
                     layer=l)
        else:
            kv, _ = om.tensor(po.KV, l)
            kv = kv.view(np.uint16).reshape(2, c["max_ctx"], nkv * hd)
            gm.adopt(g.KV, np.ascontiguousarray(kv[:, :ctx]), layer=l)
    gm.position = ctx


def rel_err(got, want):
    """max |got - want| over max |want| (the reference's gpu_check.cpp:80-94 measure)"""
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def near_tie_rows(logits, tol):
    """rows whose top-2 logit gap is below tol (greedy tokens there may legitimately differ)"""
    s = np.sort(logits, axis=1)
    return set(np.nonzero(s[:, -1] - s[:, -2] < tol)[0].tolist())


def route_margins(om, trace):
    """[n_layers][n]: the gap between the K-th and (K+1)-th router logit of each row at each layer, from the oracle's
    MoE inputs (trace[l][2]) and the layer's bf16 router; a small gap is a routing near-tie, where a perturbation of
    the row's input far below the logits' tolerance may swap an expert"""
    c = om.cfg
    K, E, H = c["top_k"], c["n_experts"], c["hidden"]
    out = []
    for l in range(c["n_layers"]):
        R = (om.tensor(po.ROUTER, l)[0].view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(E, H)
        lg = -np.sort(-(trace[l, 2].astype(np.float64) @ R.T.astype(np.float64)), axis=1)
        out.append(lg[:, K - 1] - lg[:, K])
    return np.array(out)
