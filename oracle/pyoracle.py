"""numpy bindings of the CPU oracle (liboracle.so) and of the reference built from its sources (_ref/libgeode_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the timed CPU baseline. The product (geode_amd) never imports this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libgeode_ref.so")

_c = ctypes
_P = _c.c_void_p


def _ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


def q4_row_bytes(cols):
    return cols // 16 * 9


class Config(_c.Structure):
    _fields_ = [(n, _c.c_int) for n in ("hidden", "vocab", "n_layers", "n_experts", "top_k", "moe_ff", "shared_ff",
                                        "n_heads", "n_kv_heads", "head_dim", "rope_dim")] + \
               [("rope_theta", _c.c_float), ("eps", _c.c_float), ("max_ctx", _c.c_int), ("attn_block", _c.c_int),
                ("kv_int8", _c.c_int)] + \
               [(n, _c.c_int) for n in ("gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim", "conv_kernel")] + \
               [("gdn_layers", _c.c_ubyte * 256), ("mtp", _c.c_int)]


class MoeWeights(_c.Structure):
    _fields_ = [("H", _c.c_int), ("E", _c.c_int), ("K", _c.c_int), ("F", _c.c_int), ("SF", _c.c_int),
                ("experts", _P), ("expert_globals", _P), ("sh_gate", _P), ("sh_up", _P), ("sh_down", _P),
                ("sh_globals", _c.c_float * 3), ("shared_gate", _P), ("router", _P)]


# tensor kinds, numbered as in oracle.h and include/geode_verify.h
EMBED, LM_HEAD, FINAL_NORM, IN_NORM, POST_NORM, Q, K, V, O, Q_NORM, K_NORM, ROUTER, SHARED_GATE, EXPERT, SH_GATE, \
    SH_UP, SH_DOWN, KV, KV8, KVS = range(20)
GDN_QKV, GDN_Z, GDN_OUT, GDN_A, GDN_B, GDN_ALOG, GDN_DTB, GDN_CONV, GDN_NORM, GDN_CONV_ST, GDN_S = range(20, 31)
MTP_FC, MTP_NORM, MTP_PRE_E, MTP_PRE_H = range(31, 35)


class StateInfo(_c.Structure):
    _fields_ = [("pack_print", _c.c_uint64), ("conv_id", _c.c_uint64), ("extra", _c.c_int32),
                ("rope_delta", _c.c_int32), ("has_mtp", _c.c_int32), ("has_vision", _c.c_int32), ("hidden", _P),
                ("has_hidden", _c.c_int32)]


def _load():
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("oracle/liboracle.so is not built (run __graft_entry__.build())")
    lib = _c.CDLL(LIB_PATH)
    sig = {
        "orc_hash": (_c.c_uint64, [_c.c_uint64, _c.c_uint64]),
        "orc_fill_normal": (None, [_c.c_uint64, _c.c_int64, _c.c_float, _c.c_float, _P]),
        "orc_fill_uniform": (None, [_c.c_uint64, _c.c_int64, _P]),
        "orc_f32_to_f16": (_c.c_uint16, [_c.c_float]),
        "orc_f16_to_f32": (_c.c_float, [_c.c_uint16]),
        "orc_f32_to_bf16": (_c.c_uint16, [_c.c_float]),
        "orc_set_threads": (None, [_c.c_int]),
        "orc_threads": (_c.c_int, []),
        "orc_e4m3_value": (_c.c_float, [_c.c_uint8]),
        "orc_e4m3_byte": (_c.c_uint8, [_c.c_float]),
        "orc_q4_block": (None, [_P, _c.c_float, _P, _P]),
        "orc_q4_global": (_c.c_float, [_P, _c.c_int64]),
        "orc_q4_pack": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P]),
        "orc_dequant_rows": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P]),
        "orc_matvec_rows": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P, _P]),
        "orc_quantize_activation": (None, [_P, _c.c_int64, _P, _P, _P]),
        "orc_matvec_rows_q": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P, _P, _P]),
        "orc_matvec_bf16": (None, [_P, _c.c_int64, _c.c_int64, _c.c_int, _P, _P]),
        "orc_rmsnorm": (None, [_P, _P, _P, _c.c_int, _c.c_float, _c.c_int]),
        "orc_route_topk": (None, [_P, _c.c_int, _c.c_int, _P, _P]),
        "orc_ffn_swiglu": (None, [_P, _P, _P, _c.c_float, _c.c_float, _c.c_float, _c.c_int, _c.c_int, _c.c_int, _P,
                                  _c.c_int, _P]),
        "orc_moe_layer": (None, [_c.POINTER(MoeWeights), _c.c_int, _P, _P, _c.c_int, _P, _P, _P, _P]),
        "orc_quant_kv_row": (None, [_P, _c.c_int, _P, _P]),
        "orc_model_create": (_P, [_c.POINTER(Config)]),
        "orc_model_free": (None, [_P]),
        "orc_model_tensor": (_P, [_P, _c.c_int, _c.c_int, _c.c_int, _c.POINTER(_c.c_int64), _P]),
        "orc_model_fill": (None, [_P, _c.c_uint64, _c.c_float, _c.c_float, _c.c_int, _c.c_int]),
        "orc_model_set_position": (None, [_P, _c.c_int]),
        "orc_model_position": (_c.c_int, [_P]),
        "orc_model_verify": (_c.c_int, [_P, _P, _c.c_int, _P, _c.c_int, _P, _P]),
        "orc_model_verify_trace": (_c.c_int, [_P, _P, _c.c_int, _P, _c.c_int, _P, _P, _P]),
        "orc_model_keep": (_c.c_int, [_P, _c.c_int, _P]),
        "orc_model_last_times": (None, [_P, _P, _P]),
        "orc_model_hidden": (_c.c_int, [_P, _P, _c.c_int]),
        "orc_model_mtp": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _P, _c.c_int, _P]),
        "orc_model_draft": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _P, _c.c_int, _P, _P, _P]),
        "orc_model_draft_next": (_c.c_int, [_P, _c.c_int32, _c.c_int, _c.c_int, _P, _P, _P]),
        "orc_model_set_draft_vocab": (_c.c_int, [_P, _P, _c.c_int]),
        "orc_sample": (_c.c_int, [_P, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_int, _c.c_double]),
        "orc_sample_seeded": (None, [_P, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_uint64, _c.c_int, _P]),
        "orc_accept_match": (_c.c_int, [_P, _c.c_int, _P, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_int, _P,
                                        _P, _P]),
        "orc_accept_match_ex": (_c.c_int, [_P, _c.c_int, _P, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_int,
                                           _P, _P, _c.c_int, _c.c_float, _P, _c.c_int, _P, _P]),
        "orc_accept_textbook": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _P, _P,
                                           _c.c_float, _P]),
        "orc_nucleus_probs": (None, [_P, _c.c_int, _c.c_float, _c.c_float, _P]),
        "orc_fnv1a": (_c.c_uint64, [_P, _c.c_size_t, _c.c_uint64]),
        "orc_fast_exp": (_c.c_float, [_c.c_float]),
        "orc_gdn_step": (None, [_P, _c.c_int, _c.c_int, _P, _P, _P, _c.c_float, _c.c_float, _P]),
        "orc_model_config": (_P, [_P]),
        "orc_state_save": (_c.c_int, [_P, _c.c_char_p, _c.c_int, _c.POINTER(StateInfo), _c.c_char_p, _c.c_int]),
        "orc_state_load": (_c.c_int, [_P, _c.c_char_p, _c.POINTER(StateInfo), _c.c_char_p, _c.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def load_ref():
    """The reference's own functions (oracle/_ref), or None where they were not built (e.g. on the GPU box)."""
    if not os.path.exists(REF_PATH):
        return None
    r = _c.CDLL(REF_PATH)
    sig = {
        "ref_e4m3_value": (_c.c_float, [_c.c_uint8]),
        "ref_e4m3_byte": (_c.c_uint8, [_c.c_float]),
        "ref_q4_block": (None, [_P, _c.c_float, _P, _P]),
        "ref_dequant_rows": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P]),
        "ref_matvec_rows": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P, _P]),
        "ref_quantize_activation": (None, [_P, _c.c_int64, _P, _P, _P]),
        "ref_matvec_rows_q": (None, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P, _P]),
        "ref_matvec_bf16_multi": (None, [_P, _c.c_int64, _c.c_int64, _c.c_int, _P, _P]),
        "ref_rmsnorm": (None, [_P, _P, _P, _c.c_int, _c.c_float, _c.c_int]),
        "ref_sample_seeded": (None, [_P, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_uint64, _c.c_int, _P]),
        "ref_to_tile8": (None, [_c.c_int64, _c.c_int64, _P, _P]),
        "ref_tile8_row": (None, [_P, _c.c_int64, _c.c_int64, _c.c_int64, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(r, name)
        f.restype = res
        f.argtypes = args
    return r


# ---------------------------------------------------------------- numpy wrappers
def normal(seed, n, sigma=1.0, mean=0.0):
    out = np.empty(int(n), np.float32)
    lib.orc_fill_normal(seed, int(n), mean, sigma, _ptr(out))
    return out


def uniform(seed, n):
    out = np.empty(int(n), np.float32)
    lib.orc_fill_uniform(seed, int(n), _ptr(out))
    return out


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    return np.array([lib.orc_f32_to_f16(float(v)) for v in x.ravel()], np.uint16).reshape(x.shape)


def q4_pack(w):
    """fp32 [rows, cols] -> (pack-layout bytes [rows, cols/16*9], global s2)"""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    s2 = lib.orc_q4_global(_ptr(w), w.size)
    out = np.empty((rows, q4_row_bytes(cols)), np.uint8)
    lib.orc_q4_pack(_ptr(w), rows, cols, s2, _ptr(out))
    return out, s2


def q4_random(seed, rows, cols, sigma=0.02):
    return q4_pack(normal(seed, rows * cols, sigma).reshape(rows, cols))


def dequant(wq, cols, g):
    rows = wq.shape[0]
    out = np.empty((rows, cols), np.float32)
    lib.orc_dequant_rows(_ptr(np.ascontiguousarray(wq)), rows, cols, g, _ptr(out))
    return out


def matvec(wq, cols, g, x):
    rows = wq.shape[0]
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    lib.orc_matvec_rows(_ptr(np.ascontiguousarray(wq)), rows, cols, g, _ptr(x), _ptr(y))
    return y


def quantize_activation(x):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.size
    q = np.empty(cols, np.int8)
    s = np.empty(cols // 16, np.float32)
    b = np.empty(cols // 16, np.int32)
    lib.orc_quantize_activation(_ptr(x), cols, _ptr(q), _ptr(s), _ptr(b))
    return q, s, b


def matvec_q(wq, cols, g, x):
    q, s, _ = quantize_activation(x)
    rows = wq.shape[0]
    y = np.empty(rows, np.float32)
    lib.orc_matvec_rows_q(_ptr(np.ascontiguousarray(wq)), rows, cols, g, _ptr(q), _ptr(s), _ptr(y))
    return y


def matvec_bf16(w, x):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = w.shape
    n = x.shape[0]
    y = np.empty((n, rows), np.float32)
    lib.orc_matvec_bf16(_ptr(w), rows, cols, n, _ptr(x), _ptr(y))
    return y


def rmsnorm(x, w, eps=1e-6, zero_centered=True):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib.orc_rmsnorm(_ptr(x), _ptr(np.ascontiguousarray(w, np.float32)) if w is not None else None, _ptr(out), x.size,
                    eps, int(zero_centered))
    return out


def quant_kv_row(x):
    """(int8 row, scale) as quant_kv_row makes them (model.cpp:3766-3774)"""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.size, np.int8)
    s = np.zeros(1, np.float32)
    lib.orc_quant_kv_row(_ptr(x), x.size, _ptr(q), _ptr(s))
    return q, float(s[0])


def route_topk(logits, K):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    lib.orc_route_topk(_ptr(logits), logits.size, K, _ptr(ids), _ptr(w))
    return ids, w


def ffn_swiglu(gate, up, down, gg, gu, gd, H, F, x_f16, mode=0):
    M = x_f16.shape[0]
    y = np.empty((M, H), np.float32)
    lib.orc_ffn_swiglu(_ptr(gate), _ptr(up), _ptr(down), gg, gu, gd, H, F, M,
                       _ptr(np.ascontiguousarray(x_f16, np.uint16)), mode, _ptr(y))
    return y


def moe_layer(model, layer, h, router_logits=None, mode=0):
    """orc_moe_layer on the oracle model's layer weights: (out [M][H] without the residual, ids, weights)"""
    c = model.cfg
    H, E, K, F = c["hidden"], c["n_experts"], c["top_k"], c["moe_ff"]
    blocks, globs = [], []
    for e in range(E):
        b, g = model.tensor(EXPERT, layer, e)
        blocks.append(b)
        globs.append(np.asarray(g[:2], np.float32))
    experts = np.ascontiguousarray(np.concatenate(blocks))
    eg = np.ascontiguousarray(np.concatenate(globs), np.float32)
    sg, gsg = model.tensor(SH_GATE, layer)
    su, gsu = model.tensor(SH_UP, layer)
    sd, gsd = model.tensor(SH_DOWN, layer)
    shared_gate = np.ascontiguousarray(model.tensor(SHARED_GATE, layer)[0])
    router = np.ascontiguousarray(model.tensor(ROUTER, layer)[0])
    w = MoeWeights(H, E, K, F, c["shared_ff"], _ptr(experts), _ptr(eg), _ptr(sg), _ptr(su), _ptr(sd),
                   (_c.c_float * 3)(gsg[0], gsu[0], gsd[0]), _ptr(shared_gate), _ptr(router))
    h = np.ascontiguousarray(h, np.float32)
    M = h.shape[0]
    out = np.empty((M, H), np.float32)
    ids = np.empty((M, K), np.int32)
    wts = np.empty((M, K), np.float32)
    lg = np.ascontiguousarray(router_logits, np.float32) if router_logits is not None else None
    lib.orc_moe_layer(_c.byref(w), M, _ptr(h), _ptr(lg) if lg is not None else None, mode, _ptr(out), _ptr(ids),
                      _ptr(wts), None)
    return out, ids, wts


def sample(logits, temperature, top_p, top_k=0, cap=1024, u=0.5):
    logits = np.ascontiguousarray(logits, np.float32)
    return lib.orc_sample(_ptr(logits), logits.size, temperature, top_p, top_k, cap, u)


def nucleus_probs(logits, temperature, top_p):
    logits = np.ascontiguousarray(logits, np.float32)
    p = np.empty(logits.size, np.float64)
    lib.orc_nucleus_probs(_ptr(logits), logits.size, temperature, top_p, _ptr(p))
    return p


def accept_textbook(target, draft, temperature, top_p, greedy, u_draft, u_acc, u_res):
    target = np.ascontiguousarray(target, np.float32)
    draft = np.ascontiguousarray(draft, np.float32)
    k, V = draft.shape
    out = np.empty(k + 1, np.int32)
    n = lib.orc_accept_textbook(_ptr(target), _ptr(draft), V, k, temperature, top_p, int(greedy),
                                _ptr(np.ascontiguousarray(u_draft, np.float32)),
                                _ptr(np.ascontiguousarray(u_acc, np.float32)), float(u_res), _ptr(out))
    return out[:n]


def accept_match(logits, batch, temperature, top_p, top_k=0, cap=1024, u=None):
    logits = np.ascontiguousarray(logits, np.float32)
    n, V = logits.shape
    u = np.ascontiguousarray(u if u is not None else np.full(n, 0.5), np.float64)
    out = np.empty(n, np.int32)
    kept = _c.c_int(0)
    cnt = lib.orc_accept_match(_ptr(logits), V, _ptr(np.ascontiguousarray(batch, np.int32)), n, temperature, top_p,
                               top_k, cap, _ptr(u), _ptr(out), _c.byref(kept))
    return out[:cnt], kept.value


def accept_match_ex(logits, batch, temperature, top_p, top_k=0, cap=1024, u=None, seen=(), presence_penalty=0.0,
                    stop=()):
    """sample-and-match with the presence penalty and stop tokens: (emitted tokens, kept rows, the penalized logits)"""
    lg = np.array(logits, np.float32, copy=True, order="C")
    n, V = lg.shape
    u = np.ascontiguousarray(u if u is not None else np.full(n, 0.5), np.float64)
    sn = np.ascontiguousarray(np.asarray(seen, np.int32).reshape(-1))
    st = np.ascontiguousarray(np.asarray(stop, np.int32).reshape(-1))
    out = np.empty(n, np.int32)
    kept = _c.c_int(0)
    cnt = lib.orc_accept_match_ex(_ptr(lg), V, _ptr(np.ascontiguousarray(batch, np.int32)), n, temperature, top_p,
                                  top_k, cap, _ptr(u), _ptr(sn), sn.size, presence_penalty, _ptr(st), st.size,
                                  _ptr(out), _c.byref(kept))
    return out[:cnt], kept.value, lg


class Model:
    """The oracle's whole model (orc_model_*): host-side weights in the pack layout."""

    def __init__(self, cfg: dict, seed=1, sigma=0.02, router_sigma=0.0221, ctx=0, fast=False):
        self.cfg = dict(cfg)
        c = Config(**{k: cfg[k] for k, _ in Config._fields_ if k in cfg and k != "gdn_layers"})
        for l, g in enumerate(cfg.get("gdn_layers", ())):
            c.gdn_layers[l] = 1 if g else 0
        if "attn_block" not in cfg:
            c.attn_block = 1024
        self._c = c
        self.h = lib.orc_model_create(_c.byref(c))
        lib.orc_model_fill(self.h, seed, sigma, router_sigma, ctx, int(fast))

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_model_free(self.h)
            self.h = None

    def tensor(self, kind, layer=0, expert=0):
        """(numpy uint8 view of the bytes, globals[2])"""
        nb = _c.c_int64(0)
        g = np.zeros(2, np.float32)
        p = lib.orc_model_tensor(self.h, kind, layer, expert, _c.byref(nb), _ptr(g))
        if not p:
            raise KeyError((kind, layer, expert))
        buf = (_c.c_uint8 * nb.value).from_address(p)
        return np.frombuffer(buf, np.uint8), g

    @property
    def position(self):
        return lib.orc_model_position(self.h)

    @position.setter
    def position(self, p):
        lib.orc_model_set_position(self.h, p)

    def verify(self, tokens, parents=None, mode=0, route=False):
        tokens = np.ascontiguousarray(tokens, np.int32)
        n = tokens.size
        logits = np.empty((n, self.cfg["vocab"]), np.float32)
        par = np.ascontiguousarray(parents, np.int32) if parents is not None else None
        ids = np.empty((self.cfg["n_layers"], n, self.cfg["top_k"]), np.int32) if route else None
        rc = lib.orc_model_verify(self.h, _ptr(tokens), n, _ptr(par), mode, _ptr(logits), _ptr(ids))
        if rc != 0:
            raise ValueError("orc_model_verify failed")
        return (logits, ids) if route else logits

    def verify_trace(self, tokens, parents=None, mode=0):
        """(logits, route ids [L][n][K], trace [L][4][n][hidden]: per layer the residual stream in, after the
        attention's residual add, the MoE block's input (post-norm) and the MoE block's output)"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        n = tokens.size
        c = self.cfg
        logits = np.empty((n, c["vocab"]), np.float32)
        par = np.ascontiguousarray(parents, np.int32) if parents is not None else None
        ids = np.empty((c["n_layers"], n, c["top_k"]), np.int32)
        tr = np.empty((c["n_layers"], 4, n, c["hidden"]), np.float32)
        if lib.orc_model_verify_trace(self.h, _ptr(tokens), n, _ptr(par), mode, _ptr(logits), _ptr(ids), _ptr(tr)):
            raise ValueError("orc_model_verify_trace failed")
        return logits, ids, tr

    def keep(self, kept, path=None):
        p = np.ascontiguousarray(path, np.int32) if path is not None else None
        if lib.orc_model_keep(self.h, kept, _ptr(p)) != 0:
            raise ValueError("orc_model_keep failed")

    def hidden(self):
        """the last verify's rows after the final norm [n][hidden] (the MTP layer's input)"""
        rows = self.cfg.get("max_rows", 32)
        out = np.empty((rows, self.cfg["hidden"]), np.float32)
        n = lib.orc_model_hidden(self.h, _ptr(out), rows)
        return out[:n].copy()

    def _draft_rows(self):
        return len(self._draft_ids) if getattr(self, "_draft_ids", None) is not None else self.cfg["vocab"]

    def set_draft_vocab(self, ids):
        """the draft head: lm_head's rows of ids (None or empty: the whole vocabulary)"""
        a = np.ascontiguousarray(ids if ids is not None else [], np.int32)
        if lib.orc_model_set_draft_vocab(self.h, _ptr(a), a.size) != 0:
            raise ValueError("orc_model_set_draft_vocab failed")
        self._draft_ids = a if a.size else None

    def mtp(self, tokens, pos, hidden=None, mode=0, logits=True):
        """forward_mtp: the last row's logits over the draft head (None when logits=False: the KV only)"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        hid = np.ascontiguousarray(hidden, np.float32) if hidden is not None else None
        lg = np.empty(self._draft_rows(), np.float32) if logits else None
        if lib.orc_model_mtp(self.h, _ptr(tokens), tokens.size, pos, _ptr(hid), mode, _ptr(lg)) != 0:
            raise ValueError("orc_model_mtp failed")
        return lg

    def draft(self, tokens, pos, hidden=None, mode=0):
        """Model::draft: (draft token, its probability, the last row's logits)"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        hid = np.ascontiguousarray(hidden, np.float32) if hidden is not None else None
        lg = np.empty(self._draft_rows(), np.float32)
        d, p = _c.c_int32(0), _c.c_float(0)
        if lib.orc_model_draft(self.h, _ptr(tokens), tokens.size, pos, _ptr(hid), mode, _ptr(lg), _c.byref(d),
                               _c.byref(p)) != 0:
            raise ValueError("orc_model_draft failed")
        return d.value, p.value, lg

    def draft_next(self, token, pos, mode=0):
        """Model::draft_next: (draft token, its probability, logits) from the last MTP pass's output"""
        lg = np.empty(self._draft_rows(), np.float32)
        d, p = _c.c_int32(0), _c.c_float(0)
        if lib.orc_model_draft_next(self.h, int(token), pos, mode, _ptr(lg), _c.byref(d), _c.byref(p)) != 0:
            raise ValueError("orc_model_draft_next failed")
        return d.value, p.value, lg

    def save_state(self, path, append=False, *, pack_print=0, conv_id=0, extra=0, rope_delta=0, has_mtp=False,
                   has_vision=False, hidden=None):
        """orc_state_save: Model::save_state (state.cpp:251-371) of this model's position and KV cache"""
        hid = np.ascontiguousarray(hidden, np.float32) if hidden is not None else None
        info = StateInfo(pack_print, conv_id, extra, rope_delta, int(has_mtp), int(has_vision), _ptr(hid), 0)
        err = _c.create_string_buffer(512)
        if lib.orc_state_save(self.h, os.fsencode(path), int(append), _c.byref(info), err, 512) != 0:
            raise OSError(err.value.decode())

    def load_state(self, path, *, pack_print=0, has_mtp=False, has_vision=False):
        """orc_state_load: Model::load_state (state.cpp:373-463); ValueError with the reference's message on refusal"""
        hid = np.zeros(self.cfg["hidden"], np.float32)
        info = StateInfo(pack_print, 0, 0, 0, int(has_mtp), int(has_vision), _ptr(hid), 0)
        err = _c.create_string_buffer(512)
        if lib.orc_state_load(self.h, os.fsencode(path), _c.byref(info), err, 512) != 0:
            raise ValueError(err.value.decode())
        return {"conv_id": info.conv_id, "extra": info.extra, "rope_delta": info.rope_delta,
                "hidden": hid if info.has_hidden else None}

    def last_times(self):
        a, b = _c.c_double(0), _c.c_double(0)
        lib.orc_model_last_times(self.h, _c.byref(a), _c.byref(b))
        return a.value, b.value


def fast_exp(x):
    return lib.orc_fast_exp(float(x))


def gdn_step(S, q, k, v, decay, beta):
    """one token of the delta rule on one head: (new S [dk][dv], out [dv]) (orc_gdn_step)"""
    S = np.array(S, np.float32, copy=True)
    dk, dv = S.shape
    out = np.empty(dv, np.float32)
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
    lib.orc_gdn_step(_ptr(S), dk, dv, _ptr(q), _ptr(k), _ptr(v), decay, beta, _ptr(out))
    return S, out
