"""Writes a geode-pack (the format engine/src/pack.cpp:39-308 reads) from the oracle model's tensors, for the pack
loader's tests: geode.json, dense.bin (every tensor but the experts; a Gated DeltaNet layer's linear_attn.* tensors in
place of its self_attn.* ones) and experts.bin (per layer the routed experts' blocks, gate_up rows then down rows,
pack.cpp:329-333), the experts optionally in the tile8 layout
(engine/src/kernels.cpp:971-991, restated in `to_tile8` below and pinned against the reference's own to_tile8 by the
golden fixture). Tensor names and shapes as Model::bind_layer binds them (engine/src/model.cpp:95-202)."""
import json
import os

import numpy as np

import pyoracle as po


def _affine_to():
    """the pack's q4 nibble c to the affine order (kernels.cpp:907-930): c < 8 -> c + 8, else 15 - c"""
    t = np.zeros(256, np.uint8)
    for b in range(256):
        v = 0
        for k in range(2):
            c = (b >> (4 * k)) & 15
            v |= (c + 8 if c < 8 else 15 - c) << (4 * k)
        t[b] = v
    return t


AFFINE = _affine_to()


def to_tile8(rows, cols, m):
    """q4 pack rows [rows][cols / 16 * 9] in the tile8 layout: per 32-row tile, code word j of chunk c of quad i (the
    four rows' 32-bit words, affine) at ((c * 8 + j) * 8 + i) * 16 + 4 r, then the scales, block b of chunk c of row r
    of quad i at 1024 * nch + (c * 8 + i) * 16 + 4 b + r"""
    m = np.asarray(m, np.uint8).reshape(rows, cols // 16 * 9)
    nch, code = cols // 64, cols // 2
    out = np.empty_like(m).reshape(rows // 32, 32 * m.shape[1])
    for t in range(rows // 32):
        tile = m[32 * t:32 * t + 32]
        g = out[t]
        codes = AFFINE[tile[:, :code]].reshape(8, 4, nch, 8, 4)       # [quad i][row r][chunk c][word j][byte k]
        g[:1024 * nch] = codes.transpose(2, 3, 0, 1, 4).reshape(-1)   # [c][j][i][r][k]
        sc = tile[:, code:].reshape(8, 4, nch, 4)                      # [i][r][c][block b]
        g[1024 * nch:] = sc.transpose(2, 0, 3, 1).reshape(-1)          # [c][i][b][r]
    return out.reshape(rows, -1)


class _Bin:
    def __init__(self):
        self.parts, self.size = [], 0

    def add(self, data):
        b = np.ascontiguousarray(data).tobytes()
        off = self.size
        self.parts.append(b)
        self.size += len(b)
        pad = (-self.size) % 64   # (64-byte aligned tensors, as a real pack's)
        if pad:
            self.parts.append(b"\0" * pad)
            self.size += pad
        return off

    def write(self, path):
        with open(path, "wb") as f:
            for p in self.parts:
                f.write(p)


def write_pack(om, directory, tile8=False, extra_config=None, mutate=None, draft_vocab=None):
    """The oracle model om as a pack in directory; returns the manifest (dict). mutate(manifest) may damage it before
    it is written (the refusal tests). A model with an MTP layer: its tensors under mtp.* (model.cpp:175-191) and the
    manifest's "mtp" object with its experts (pack.cpp:303-305); draft_vocab: token ids for draft_vocab.bin."""
    os.makedirs(directory, exist_ok=True)
    c = om.cfg
    H, V, L, E = c["hidden"], c["vocab"], c["n_layers"], c["n_experts"]
    nh, nkv, hd, F = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["moe_ff"]
    dense, experts = _Bin(), _Bin()
    tensors = {}

    def put(name, dtype, shape, data, glob=None):
        t = {"type": dtype, "shape": list(shape), "file": "dense.bin", "offset": dense.add(data)}
        if glob is not None:
            t["global"] = float(glob)
        tensors[name] = t

    t, g = om.tensor(po.EMBED)
    put("embed_tokens.weight", "q4", (V, H), t, g[0])
    t, g = om.tensor(po.LM_HEAD)
    put("lm_head.weight", "q4", (V, H), t, g[0])
    put("norm.weight", "f32", (H,), om.tensor(po.FINAL_NORM)[0])
    layers = []
    gdn = c.get("gdn_layers", ())

    def layer(l, p):
        put(p + "input_layernorm.weight", "f32", (H,), om.tensor(po.IN_NORM, l)[0])
        put(p + "post_attention_layernorm.weight", "f32", (H,), om.tensor(po.POST_NORM, l)[0])
        if l < L and l < len(gdn) and gdn[l]:   # a Gated DeltaNet layer (Model::bind_layer, model.cpp:136-146)
            nk, nv, dk, dv, K = c["gdn_k_heads"], c["gdn_v_heads"], c["gdn_k_dim"], c["gdn_v_dim"], c["conv_kernel"]
            conv_dim, vd = 2 * nk * dk + nv * dv, nv * dv
            for kind, name, shape in ((po.GDN_QKV, "in_proj_qkv", (conv_dim, H)), (po.GDN_Z, "in_proj_z", (vd, H)),
                                      (po.GDN_OUT, "out_proj", (H, vd))):
                t, g = om.tensor(kind, l)
                put(p + f"linear_attn.{name}.weight", "q4", shape, t, g[0])
            put(p + "linear_attn.in_proj_a.weight", "bf16", (nv, H), om.tensor(po.GDN_A, l)[0])
            put(p + "linear_attn.in_proj_b.weight", "bf16", (nv, H), om.tensor(po.GDN_B, l)[0])
            put(p + "linear_attn.A_log", "f32", (nv,), om.tensor(po.GDN_ALOG, l)[0])
            put(p + "linear_attn.dt_bias", "f32", (nv,), om.tensor(po.GDN_DTB, l)[0])
            put(p + "linear_attn.conv1d.weight", "f32", (conv_dim, 1, K), om.tensor(po.GDN_CONV, l)[0])
            put(p + "linear_attn.norm.weight", "f32", (dv,), om.tensor(po.GDN_NORM, l)[0])
        else:
            for kind, name, rows in ((po.Q, "q_proj", nh * hd * 2), (po.K, "k_proj", nkv * hd),
                                     (po.V, "v_proj", nkv * hd)):
                t, g = om.tensor(kind, l)
                put(p + f"self_attn.{name}.weight", "q4", (rows, H), t, g[0])
            t, g = om.tensor(po.O, l)
            put(p + "self_attn.o_proj.weight", "q4", (H, nh * hd), t, g[0])
            put(p + "self_attn.q_norm.weight", "f32", (hd,), om.tensor(po.Q_NORM, l)[0])
            put(p + "self_attn.k_norm.weight", "f32", (hd,), om.tensor(po.K_NORM, l)[0])
        put(p + "mlp.gate.weight", "bf16", (E, H), om.tensor(po.ROUTER, l)[0])
        put(p + "mlp.shared_expert_gate.weight", "bf16", (1, H), om.tensor(po.SHARED_GATE, l)[0])
        for kind, name, shape in ((po.SH_GATE, "gate_proj", (F, H)), (po.SH_UP, "up_proj", (F, H)),
                                  (po.SH_DOWN, "down_proj", (H, F))):
            t, g = om.tensor(kind, l)
            put(p + f"mlp.shared_expert.{name}.weight", "q4", shape, t, g[0])
        scales = np.zeros((E, 2), np.float32)
        gu_bytes = 2 * F * (H // 16 * 9)
        first = None
        for e in range(E):
            blk, g = om.tensor(po.EXPERT, l, e)
            scales[e] = g[:2]
            if tile8:
                blk = np.concatenate([to_tile8(2 * F, H, blk[:gu_bytes]).reshape(-1),
                                      to_tile8(H, F, blk[gu_bytes:]).reshape(-1)])
            off = experts.add(blk)
            first = off if first is None else first
        stride = (gu_bytes + H * (F // 16 * 9) + 63) // 64 * 64
        put(p + "mlp.experts.scales", "f32", (E, 2), scales)
        return {"file": "experts.bin", "offset": first, "stride": stride, "format": "q4"}

    for l in range(L):
        layers.append(layer(l, f"layers.{l}."))
    mtp = None
    if c.get("mtp"):
        mtp = {"experts": layer(L, "mtp.layers.0.")}
        t, g = om.tensor(po.MTP_FC)
        put("mtp.fc.weight", "q4", (H, 2 * H), t, g[0])
        for kind, name in ((po.MTP_NORM, "norm"), (po.MTP_PRE_E, "pre_fc_norm_embedding"),
                           (po.MTP_PRE_H, "pre_fc_norm_hidden")):
            put(f"mtp.{name}.weight", "f32", (H,), om.tensor(kind)[0])
    if draft_vocab is not None:
        np.asarray(draft_vocab, "<i4").tofile(os.path.join(directory, "draft_vocab.bin"))
    config = {"hidden_size": H, "num_hidden_layers": L, "vocab_size": V, "rms_norm_eps": c["eps"],
              "num_attention_heads": nh, "num_key_value_heads": nkv, "head_dim": hd,
              "rope_parameters": {"rope_theta": c["rope_theta"], "partial_rotary_factor": c["rope_dim"] / hd},
              "num_experts": E, "num_experts_per_tok": c["top_k"], "moe_intermediate_size": F,
              "shared_expert_intermediate_size": c["shared_ff"],
              "layer_types": ["linear_attention" if l < len(gdn) and gdn[l] else "full_attention" for l in range(L)]}
    if any(gdn):
        config.update({"linear_num_key_heads": c["gdn_k_heads"], "linear_num_value_heads": c["gdn_v_heads"],
                       "linear_key_head_dim": c["gdn_k_dim"], "linear_value_head_dim": c["gdn_v_dim"],
                       "linear_conv_kernel_dim": c["conv_kernel"]})
    config.update(extra_config or {})
    dense.write(os.path.join(directory, "dense.bin"))
    experts.write(os.path.join(directory, "experts.bin"))
    m = {"format": "geode-pack", "version": 1, "arch": "qwen35moe",
         "files": [{"name": "dense.bin", "size": dense.size}, {"name": "experts.bin", "size": experts.size}],
         "config": config, "tensors": tensors, "experts": {"layers": layers},
         "formats": {"q4": {"layout": "tile8" if tile8 else "rows"}}}
    if mtp:
        m["mtp"] = mtp
    if mutate:
        mutate(m)
    with open(os.path.join(directory, "geode.json"), "w") as f:
        json.dump(m, f, indent=1)
    return m
