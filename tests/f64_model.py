"""A float64 numpy restatement of the verify step's forward pass, written from the reference's definitions, as the
independent check of the CPU oracle's layer functions (oracle/oracle_layers.cpp). Test infrastructure only.

It shares nothing with the oracle but the seeded weights (read back through pyoracle.Model.tensor) and the
dequantization of the q4 bytes (orc_dequant_rows, itself pinned bit for bit against the reference's dequant_row):
every layer step is re-derived here in float64 from the reference's formulas (paths under engine/src/):

* RMSNorm with a (1 + w) weight: x / sqrt(mean(x^2) + eps) * (1 + w)                      kernels.cpp:1520-1529
* attention (model.cpp:3690-4019): q_proj rows per head [query hd | gate hd]; per-head RMSNorm(1 + w) of the
  query and key; partial RoPE on the first rope_dim dims, pairs (i, i + rope_dim/2), angle pos * theta^(-2i/rope_dim)
  (:739-740, :3714-3733); keys and values stored as fp16 (attend<_Float16>, :3748-3763); scores q.k / sqrt(hd),
  softmax over the visible positions, the weighted values times sigmoid(gate) (:3852); then o_proj.
* MoE (model.cpp:4021-4065, :4123-4587): router logits = bf16 rows . h; softmax; top-K by probability (ties to the
  lower index); weights p_k / sum of the top K; experts gate_up [gate F | up F] then silu(gate) * up then down;
  the shared expert's SwiGLU times sigmoid(bf16 gate . h); out = shared + sum_k w_k y_k.
* the int8 path (mode 0): each product's input quantized per 16 values as quantize_activation does
  (kernels.cpp:1254-1295: q = clamp(nearbyint(x * 127 / amax)), value q * amax / 127); the products then in
  float64. Mode 1: the exact path, fp32 inputs (model.cpp:3337-3361).

`mistakes` plants one deliberate error in this restatement, to show that the comparison with the oracle fails for
it (each entry of MISTAKES is a plausible slip in the composition).
"""
import numpy as np

import pyoracle as po

MISTAKES = (
    "no_score_scale",      # scores q.k without 1/sqrt(hd)
    "rope_sign",           # the rotation's sine with the wrong sign
    "rope_adjacent",       # RoPE pairs (2i, 2i+1) instead of (i, i + half)
    "no_attn_gate",        # the attention output without sigmoid(gate)
    "qk_norm_plain_w",     # the q/k norm scaled by w instead of (1 + w)
    "rope_before_norm",    # RoPE applied before the q/k norm
    "no_shared_gate",      # the shared expert without its sigmoid gate
    "no_renorm",           # routed weights p_k without dividing by their sum
    "silu_wrong",          # silu(x) = x * sigmoid(-x)
    "no_causal",           # every row sees every new row (no causal / tree mask)
    "kv_f32",              # the new keys and values kept in fp32 instead of fp16
)
# slips in a Gated DeltaNet layer (model.cpp:3526-3688)
GDN_MISTAKES = (
    "gdn_no_decay",        # the state not decayed (decay 1)
    "gdn_no_beta",         # the delta's step size dropped (beta 1)
    "gdn_softplus",        # the decay's exp(-exp(A_log) (a + dt_bias)) without the softplus
    "gdn_conv_reversed",   # the conv's taps in reverse order (newest input on the oldest tap)
    "gdn_no_l2norm",       # q and k not L2-normalised
    "gdn_no_qscale",       # q without 1/sqrt(dk)
    "gdn_no_gate",         # the output's RMSNorm without the silu(z) gate
    "gdn_state_reset",     # every row from the layer's state instead of its parent's
)


def _f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def _bf16(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _rms(x, w, eps, plain=False):
    x = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * (w if plain else (1.0 + w))


def _quant(x):
    """the int8 path's activation values q * amax / 127 per 16-value block (float64 arithmetic on fp32 inputs)"""
    x32 = np.asarray(x, np.float32).astype(np.float64)
    b = x32.reshape(*x32.shape[:-1], -1, 16)
    amax = np.abs(b).max(axis=-1, keepdims=True)
    inv = np.where(amax > 0, 127.0 / np.where(amax > 0, amax, 1.0), 0.0)
    q = np.clip(np.rint(b * inv), -127, 127)
    return (q * amax / 127.0).reshape(x32.shape)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class F64Model:
    """The oracle model's weights, dequantized once, and the forward pass in float64."""

    def __init__(self, om):
        c = self.c = om.cfg
        H, V, F, hd, nh, nkv = c["hidden"], c["vocab"], c["moe_ff"], c["head_dim"], c["n_heads"], c["n_kv_heads"]
        self.om = om

        def q4(kind, rows, cols, layer=0, expert=0, which=0):
            t, g = om.tensor(kind, layer, expert)
            return po.dequant(t.reshape(rows, -1), cols, float(g[which])).astype(np.float64)

        self.embed = q4(po.EMBED, V, H)
        self.lm = q4(po.LM_HEAD, V, H)
        self.final_norm = om.tensor(po.FINAL_NORM)[0].view(np.float32).astype(np.float64)
        self.q4 = q4
        self.layers = [self._layer(l) for l in range(c["n_layers"])]
        self.mtp_layer = None
        if c.get("mtp"):   # the MTP layer (model.cpp:175-191): fc, its norms, a decoder layer at index n_layers
            self.mtp_layer = self._layer(c["n_layers"])
            self.mtp_fc = q4(po.MTP_FC, H, 2 * H)
            f32 = lambda kind: om.tensor(kind)[0].view(np.float32).astype(np.float64)   # noqa: E731
            self.mtp_norm, self.pre_e, self.pre_h = f32(po.MTP_NORM), f32(po.MTP_PRE_E), f32(po.MTP_PRE_H)
            self.mtp_out = None

    def _layer(self, l):
        c, om, q4 = self.c, self.om, self.q4
        H, F, hd, nh, nkv = c["hidden"], c["moe_ff"], c["head_dim"], c["n_heads"], c["n_kv_heads"]
        gu_bytes = 2 * F * po.q4_row_bytes(H)
        L = {}
        for k, name in ((po.IN_NORM, "in"), (po.POST_NORM, "post"), (po.Q_NORM, "qn"), (po.K_NORM, "kn")):
            L[name] = om.tensor(k, l)[0].view(np.float32).astype(np.float64)
        L["q"] = q4(po.Q, nh * 2 * hd, H, l)
        L["k"] = q4(po.K, nkv * hd, H, l)
        L["v"] = q4(po.V, nkv * hd, H, l)
        L["o"] = q4(po.O, H, nh * hd, l)
        L["router"] = _bf16(om.tensor(po.ROUTER, l)[0].view(np.uint16)).reshape(c["n_experts"], H)
        L["sgate"] = _bf16(om.tensor(po.SHARED_GATE, l)[0].view(np.uint16))
        gu, dn = [], []
        for e in range(c["n_experts"]):
            blk, g = om.tensor(po.EXPERT, l, e)
            gu.append(po.dequant(blk[:gu_bytes].reshape(2 * F, -1), H, float(g[0])).astype(np.float64))
            dn.append(po.dequant(blk[gu_bytes:].reshape(H, -1), F, float(g[1])).astype(np.float64))
        L["gu"], L["dn"] = np.stack(gu), np.stack(dn)
        SF = c["shared_ff"]
        L["sg"] = q4(po.SH_GATE, SF, H, l)
        L["su"] = q4(po.SH_UP, SF, H, l)
        L["sd"] = q4(po.SH_DOWN, H, SF, l)
        kv = om.tensor(po.KV, l)[0].view(np.float16).astype(np.float64).reshape(2, c["max_ctx"], nkv * hd)
        L["kcache"], L["vcache"] = kv[0].copy(), kv[1].copy()
        L["gdn"] = bool(c.get("gdn_layers") and l < c["n_layers"] and c["gdn_layers"][l])
        if L["gdn"]:
            nk, nv, dk, dv, K = (c["gdn_k_heads"], c["gdn_v_heads"], c["gdn_k_dim"], c["gdn_v_dim"],
                                 c["conv_kernel"])
            cd, vd = 2 * nk * dk + nv * dv, nv * dv
            f32 = lambda kind: om.tensor(kind, l)[0].view(np.float32).astype(np.float64)   # noqa: E731
            L["gqkv"] = q4(po.GDN_QKV, cd, H, l)
            L["gz"] = q4(po.GDN_Z, vd, H, l)
            L["gout"] = q4(po.GDN_OUT, H, vd, l)
            L["ga"] = _bf16(om.tensor(po.GDN_A, l)[0].view(np.uint16)).reshape(nv, H)
            L["gb"] = _bf16(om.tensor(po.GDN_B, l)[0].view(np.uint16)).reshape(nv, H)
            L["alog"], L["dtb"], L["gnorm"] = f32(po.GDN_ALOG), f32(po.GDN_DTB), f32(po.GDN_NORM)
            L["convw"] = f32(po.GDN_CONV).reshape(cd, K)
            L["conv"] = f32(po.GDN_CONV_ST).reshape(cd, K - 1)
            L["S"] = f32(po.GDN_S).reshape(nv, dk, dv)
        return L

    def _mm(self, W, x, mode):
        return (_quant(x) if mode == 0 else np.asarray(x, np.float32).astype(np.float64)) @ W.T

    def attention(self, L, h, pos, parents, mode, mistakes=()):
        c = self.c
        nh, nkv, hd, half = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["rope_dim"] // 2
        n = h.shape[0]
        q = self._mm(L["q"], h, mode).reshape(n, nh, 2 * hd)
        k = self._mm(L["k"], h, mode).reshape(n, nkv, hd)
        v = self._mm(L["v"], h, mode).reshape(n, nkv, hd)
        gate = q[:, :, hd:]
        depth = np.zeros(n, int)
        vis = np.zeros((n, n), bool)
        for i in range(n):
            if parents is None:
                depth[i] = i
                vis[i, :i + 1] = True
            else:
                depth[i] = 0 if i == 0 else depth[parents[i]] + 1
                j = i
                while j >= 0:
                    vis[i, j] = True
                    j = parents[j] if j > 0 else -1
        if "no_causal" in mistakes:
            vis[:] = True
        inv_freq = float(c["rope_theta"]) ** (-2.0 * np.arange(half) / c["rope_dim"])
        plain = "qk_norm_plain_w" in mistakes

        def rope(x, p):
            ang = p * inv_freq
            cs, sn = np.cos(ang), np.sin(ang)
            if "rope_sign" in mistakes:
                sn = -sn
            y = x.copy()
            if "rope_adjacent" in mistakes:
                a, b = x[..., 0:2 * half:2], x[..., 1:2 * half:2]
                y[..., 0:2 * half:2] = a * cs - b * sn
                y[..., 1:2 * half:2] = b * cs + a * sn
            else:
                a, b = x[..., :half], x[..., half:2 * half]
                y[..., :half] = a * cs - b * sn
                y[..., half:2 * half] = b * cs + a * sn
            return y

        qr = np.empty((n, nh, hd))
        kr = np.empty((n, nkv, hd))
        for t in range(n):
            p = pos + depth[t]
            if "rope_before_norm" in mistakes:
                qr[t] = _rms(rope(q[t, :, :hd], p), L["qn"], c["eps"], plain)
                kr[t] = _rms(rope(k[t], p), L["kn"], c["eps"], plain)
            else:
                qr[t] = rope(_rms(q[t, :, :hd], L["qn"], c["eps"], plain), p)
                kr[t] = rope(_rms(k[t], L["kn"], c["eps"], plain), p)
        store = (lambda x: x) if "kv_f32" in mistakes else _f16
        K = L["kcache"].reshape(-1, nkv, hd)
        Vc = L["vcache"].reshape(-1, nkv, hd)
        K[pos:pos + n] = store(kr)
        Vc[pos:pos + n] = store(v)
        scale = 1.0 if "no_score_scale" in mistakes else 1.0 / np.sqrt(hd)
        core = np.empty((n, nh, hd))
        group = nh // nkv
        for t in range(n):
            seen = np.concatenate([np.arange(pos), pos + np.nonzero(vis[t])[0]])
            for hh in range(nh):
                kh = hh // group
                s = K[seen, kh] @ qr[t, hh] * scale
                w = np.exp(s - s.max())
                o = (w / w.sum()) @ Vc[seen, kh]
                core[t, hh] = o if "no_attn_gate" in mistakes else o * _sigmoid(gate[t, hh])
        return self._mm(L["o"], core.reshape(n, -1), mode)

    def gdn(self, L, h, parents, mode, mistakes=()):
        """a Gated DeltaNet layer in float64 (model.cpp:3526-3688); the layer's states move on as the oracle's do (a
        chain's last row)"""
        c = self.c
        nk, nv, dk, dv, K = c["gdn_k_heads"], c["gdn_v_heads"], c["gdn_k_dim"], c["gdn_v_dim"], c["conv_kernel"]
        kd, rep = nk * dk, nv // nk
        n = h.shape[0]
        h32 = np.asarray(h, np.float32).astype(np.float64)
        proj = self._mm(L["gqkv"], h, mode)
        z = self._mm(L["gz"], h, mode)
        a, b = h32 @ L["ga"].T, h32 @ L["gb"].T
        silu = lambda x: x * _sigmoid(x)   # noqa: E731
        convs, states, core = [], [], np.empty((n, nv * dv))
        w = L["convw"][:, ::-1] if "gdn_conv_reversed" in mistakes else L["convw"]
        for t in range(n):
            parent = (t - 1 if parents is None else parents[t])
            if "gdn_state_reset" in mistakes:
                parent = -1
            cin = L["conv"] if parent < 0 else convs[parent]
            window = np.concatenate([cin, proj[t][:, None]], axis=1)   # [ch][K]: oldest first
            convs.append(window[:, 1:])
            x = silu((window * w).sum(axis=1))
            q = x[:kd].reshape(nk, dk)
            k = x[kd:2 * kd].reshape(nk, dk)
            v = x[2 * kd:].reshape(nv, dv)
            if "gdn_no_l2norm" not in mistakes:
                q = q / np.sqrt((q * q).sum(axis=1, keepdims=True) + 1e-6)
                k = k / np.sqrt((k * k).sum(axis=1, keepdims=True) + 1e-6)
            if "gdn_no_qscale" not in mistakes:
                q = q / np.sqrt(dk)
            sp = a[t] + L["dtb"]
            if "gdn_softplus" not in mistakes:
                sp = np.where(sp > 20.0, sp, np.log1p(np.exp(sp)))
            decay = np.ones(nv) if "gdn_no_decay" in mistakes else np.exp(-np.exp(L["alog"]) * sp)
            beta = np.ones(nv) if "gdn_no_beta" in mistakes else _sigmoid(b[t])
            S = (L["S"] if parent < 0 else states[parent]).copy()
            for vh in range(nv):
                kh = vh // rep
                S[vh] *= decay[vh]
                delta = (v[vh] - S[vh].T @ k[kh]) * beta[vh]
                S[vh] += np.outer(k[kh], delta)
                o = S[vh].T @ q[kh]
                o = o / np.sqrt(np.mean(o * o) + c["eps"]) * L["gnorm"]
                core[t, vh * dv:(vh + 1) * dv] = o if "gdn_no_gate" in mistakes else o * silu(z[t, vh * dv:(vh + 1) * dv])
            states.append(S)
        L["conv"], L["S"] = convs[-1], states[-1]
        return self._mm(L["gout"], core, mode)

    def moe(self, L, h, mode, mistakes=(), logits=None):
        c = self.c
        E, K = c["n_experts"], c["top_k"]
        n = h.shape[0]
        h32 = np.asarray(h, np.float32).astype(np.float64)
        lg = h32 @ L["router"].T if logits is None else np.asarray(logits, np.float64)
        p = np.exp(lg - lg.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        silu = (lambda x: x * _sigmoid(-x)) if "silu_wrong" in mistakes else (lambda x: x * _sigmoid(x))
        out = np.empty_like(h32)
        ids = np.empty((n, K), np.int64)
        wts = np.empty((n, K))
        F = c["moe_ff"]
        for t in range(n):
            order = np.lexsort((np.arange(E), -p[t]))   # by probability, ties to the lower index
            top = order[:K]
            ids[t] = top
            wts[t] = p[t, top] if "no_renorm" in mistakes else p[t, top] / p[t, top].sum()
            sg = _sigmoid(h32[t] @ L["sgate"])
            g, u = self._mm(L["sg"], h32[t:t + 1], mode)[0], self._mm(L["su"], h32[t:t + 1], mode)[0]
            sh = self._mm(L["sd"], silu(g) * u, mode)
            o = sh if "no_shared_gate" in mistakes else sg * sh
            for kk, e in enumerate(top):
                gu = self._mm(L["gu"][e], h32[t:t + 1], mode)[0]
                y = self._mm(L["dn"][e], silu(gu[:F]) * gu[F:], mode)
                o = o + wts[t, kk] * y
            out[t] = o
        return out, ids, wts, p

    def verify(self, tokens, pos, parents=None, mode=1, mistakes=()):
        """(logits [n][V], route ids [L][n][K], router probabilities [L][n][E]); the caches take the new rows"""
        c = self.c
        x = self.embed[np.asarray(tokens)].copy()
        all_ids, all_p = [], []
        for L in self.layers:
            h = _rms(x, L["in"], c["eps"])
            if L["gdn"]:
                x = x + self.gdn(L, h, parents, mode, mistakes)
            else:
                x = x + self.attention(L, h, pos, parents, mode, mistakes)
            h2 = _rms(x, L["post"], c["eps"])
            o, ids, _, p = self.moe(L, h2, mode, mistakes)
            all_ids.append(ids)
            all_p.append(p)
            x = x + o
        hf = _rms(x, self.final_norm, c["eps"])
        self.hid = hf   # the MTP layer's input rows
        return self._mm(self.lm, hf, mode), np.array(all_ids), np.array(all_p)


MTP_MISTAKES = (
    "mtp_concat_swapped",   # fc's input [hidden | embedding] instead of [embedding | hidden]
    "mtp_pre_plain_w",      # the two input norms scaled by w instead of (1 + w)
    "mtp_no_norm",          # lm_head on the layer's output without mtp.norm
    "mtp_rope_next",        # the MTP rows rotated at pos + 1 + t (the token's position) instead of pos + t
    "mtp_first_row",        # the logits of the first row instead of the last
)


def mtp_pass(fm, tokens, pos, hidden, mode=1, mistakes=(), logits=True):
    """Model::forward_mtp (model.cpp:4965-5039) in float64: row t = (hidden row t, the token after it); the MTP
    layer's KV written at pos..; the last row's logits (and its mtp.norm output kept for a chained draft)"""
    c = fm.c
    emb = fm.embed[np.asarray(tokens)]
    plain = "mtp_pre_plain_w" in mistakes
    e = _rms(emb, fm.pre_e, c["eps"], plain)
    h = _rms(np.asarray(hidden, np.float64), fm.pre_h, c["eps"], plain)
    x = fm._mm(fm.mtp_fc, np.concatenate([h, e] if "mtp_concat_swapped" in mistakes else [e, h], axis=1), mode)
    L = fm.mtp_layer
    hin = _rms(x, L["in"], c["eps"])
    x = x + fm.attention(L, hin, pos + (1 if "mtp_rope_next" in mistakes else 0), None, mode)
    o, _, _, _ = fm.moe(L, _rms(x, L["post"], c["eps"]), mode)
    x = x + o
    if not logits:
        return None
    last = x[0] if "mtp_first_row" in mistakes else x[-1]
    hn = last if "mtp_no_norm" in mistakes else _rms(last, fm.mtp_norm, c["eps"])
    fm.mtp_out = hn
    return fm._mm(fm.lm, hn[None], mode)[0]


def topk_margin(p, K):
    """the gap between the K-th and (K+1)-th largest probability of each row (a routing near-tie when small)"""
    s = -np.sort(-p, axis=-1)
    return s[..., K - 1] - s[..., K]
