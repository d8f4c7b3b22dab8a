"""geode_amd: Geode's speculative-decoding verify step on MI355X (gfx950), behind the C ABI of libgeode_verify.so.

This module is the Python host side over that ABI (ctypes; numpy for host arrays). It loads the in-tree library
and fails loudly when it is missing: there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgeode_verify.so")

_c = ctypes
_P = _c.c_void_p


class GvQ4(_c.Structure):
    _fields_ = [("codes", _P), ("scales", _P), ("rows", _c.c_int64), ("cols", _c.c_int64), ("lanes", _c.c_int32),
                ("steps", _c.c_int32), ("global_", _c.c_float)]


class GvModelConfig(_c.Structure):
    _fields_ = [(n, _c.c_int32) for n in ("hidden", "vocab", "n_layers", "n_experts", "top_k", "moe_ff", "shared_ff",
                                          "n_heads", "n_kv_heads", "head_dim", "rope_dim")] + \
               [("rope_theta", _c.c_float), ("eps", _c.c_float), ("max_ctx", _c.c_int32), ("max_rows", _c.c_int32),
                ("kv_int8", _c.c_int32)] + \
               [(n, _c.c_int32) for n in ("gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim", "conv_kernel")] + \
               [("gdn_layers", _c.c_uint8 * 256), ("mtp", _c.c_int32), ("exact", _c.c_int32)]

    @classmethod
    def of(cls, cfg):
        """the C struct of a config dict (kv_int8, the Gated DeltaNet fields and mtp optional, gdn_layers a list of
        flags)"""
        optional = ("kv_int8", "gdn_k_heads", "gdn_v_heads", "gdn_k_dim", "gdn_v_dim", "conv_kernel", "mtp", "exact")
        c = cls(**{k: cfg.get(k, 0) if k in optional else cfg[k] for k, _ in cls._fields_ if k != "gdn_layers"})
        for l, g in enumerate(cfg.get("gdn_layers", ())):
            c.gdn_layers[l] = 1 if g else 0
        return c

    def to_dict(self):
        d = {k: getattr(self, k) for k, _ in self._fields_ if k != "gdn_layers"}
        d["gdn_layers"] = [int(self.gdn_layers[l]) for l in range(min(self.n_layers, 256))]
        return d


class GvPackTensorInfo(_c.Structure):
    _fields_ = [("type", _c.c_int32), ("rows", _c.c_int64), ("cols", _c.c_int64), ("file", _c.c_int32),
                ("offset", _c.c_uint64), ("bytes", _c.c_uint64), ("global_", _c.c_float)]


class GvStateInfo(_c.Structure):
    _fields_ = [("pack_print", _c.c_uint64), ("conv_id", _c.c_uint64), ("extra", _c.c_int32),
                ("rope_delta", _c.c_int32), ("has_mtp", _c.c_int32), ("has_vision", _c.c_int32), ("hidden", _P),
                ("has_hidden", _c.c_int32)]


# tensor kinds of gv_model_adopt
EMBED, LM_HEAD, FINAL_NORM, IN_NORM, POST_NORM, QKV, O, Q_NORM, K_NORM, ROUTER, SHARED_GATE, EXPERT, \
    SHARED_EXPERT, KV, KV_I8 = 0, 1, 2, 3, 4, 5, 8, 9, 10, 11, 12, 13, 14, 17, 18
GDN_QKV, GDN_Z, GDN_OUT, GDN_A, GDN_B, GDN_ALOG, GDN_DTB, GDN_CONV, GDN_NORM, GDN_CONV_ST, GDN_S = range(20, 31)
MTP_FC, MTP_NORM, MTP_PRE_E, MTP_PRE_H = range(31, 35)

# every symbol include/geode_verify.h declares, with its signature
SIGNATURES = {
    "gv_last_error": (_c.c_char_p, []),
    "gv_init": (_c.c_int, [_c.c_int]),
    "gv_device_count": (_c.c_int, []),
    "gv_malloc": (_P, [_c.c_size_t]),
    "gv_free": (_c.c_int, [_P]),
    "gv_memcpy_h2d": (_c.c_int, [_P, _P, _c.c_size_t]),
    "gv_memcpy_d2h": (_c.c_int, [_P, _P, _c.c_size_t]),
    "gv_memcpy_d2d": (_c.c_int, [_P, _P, _c.c_size_t]),
    "gv_memset": (_c.c_int, [_P, _c.c_int, _c.c_size_t]),
    "gv_synchronize": (_c.c_int, []),
    "gv_event_record": (_c.c_int, []),
    "gv_event_elapsed_ms": (_c.c_float, [_c.c_int, _c.c_int]),
    "gv_q4_device_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64]),
    "gv_q4_from_pack": (_c.c_int, [_P, _c.c_int64, _c.c_int64, _c.c_float, _P, _c.POINTER(GvQ4)]),
    "gv_q4_dequant": (_c.c_int, [_c.POINTER(GvQ4), _P]),
    "gv_q4_pack": (_c.c_int, [_P, _c.c_int64, _c.c_int64, _P, _P]),
    "gv_act_bytes": (_c.c_size_t, [_c.c_int64]),
    "gv_quantize": (_c.c_int, [_P, _c.c_int64, _c.c_int, _c.c_int, _P, _c.c_float, _P, _P]),
    "gv_gemv_q4": (_c.c_int, [_c.POINTER(GvQ4), _P, _c.c_int, _P, _c.c_int64, _c.c_int]),
    "gv_ffn_workspace_bytes": (_c.c_size_t, [_c.c_int64, _c.c_int64, _c.c_int]),
    "gv_ffn_swiglu": (_c.c_int, [_c.POINTER(GvQ4), _c.POINTER(GvQ4), _c.POINTER(GvQ4), _c.c_int, _P, _P, _P]),
    "gv_ffn_swiglu_noalloc": (_c.c_int, [_c.POINTER(GvQ4), _c.POINTER(GvQ4), _c.POINTER(GvQ4), _c.c_int, _P, _P]),
    "gv_open": (_P, [_c.c_int, _c.c_char_p, _c.c_int]),
    "gv_close": (None, [_P]),
    "gv_adopt_q4": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int64, _c.c_size_t, _c.c_float]),
    "gv_gemm": (_c.c_int, [_P, _c.c_int, _c.c_int, _P, _P]),
    "gv_mlp": (_c.c_int, [_P, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int, _c.c_int, _P, _P]),
    "gv_model_create": (_P, [_c.POINTER(GvModelConfig), _c.c_char_p, _c.c_int]),
    "gv_model_free": (None, [_P]),
    "gv_model_adopt": (_c.c_int, [_P, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64, _P]),
    "gv_model_randomize": (_c.c_int, [_P, _c.c_uint64, _c.c_float, _c.c_float, _c.c_int]),
    "gv_model_set_position": (_c.c_int, [_P, _c.c_int]),
    "gv_model_position": (_c.c_int, [_P]),
    "gv_verify": (_c.c_int, [_P, _P, _c.c_int, _P, _P]),
    "gv_verify_keep": (_c.c_int, [_P, _c.c_int, _P]),
    "gv_model_logits": (_P, [_P]),
    "gv_model_route_ids": (_c.c_int, [_P, _P]),
    "gv_model_time_kernel": (_c.c_int, [_P, _c.c_int]),
    "gv_model_kernel_time": (_c.c_int, [_P, _P, _P]),
    "gv_model_replay": (_c.c_int, [_P, _c.c_int, _c.c_int, _c.c_int, _P]),
    "gv_model_set_graphs": (_c.c_int, [_P, _c.c_int]),
    "gv_model_set_fused": (_c.c_int, [_P, _c.c_int]),
    "gv_model_trace": (_c.c_int, [_P, _c.c_int]),
    "gv_model_trace_read": (_c.c_int64, [_P, _P, _c.c_int64]),
    "gv_model_moe": (_c.c_int, [_P, _c.c_int, _P, _c.c_int, _P, _P, _P, _P]),
    "gv_model_moe_replay": (_c.c_int, [_P, _c.c_int, _P]),
    "gv_model_layer": (_c.c_int, [_P, _c.c_int, _P, _c.c_int, _P, _P, _P, _P]),
    "gv_model_gdn_state": (_c.c_int, [_P, _c.c_int, _P, _P]),
    "gv_model_draft": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _P, _P, _P]),
    "gv_model_draft_next": (_c.c_int, [_P, _c.c_int32, _c.c_int, _P, _P]),
    "gv_model_draft_chain": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _P, _c.c_int, _c.c_float, _P, _P, _P]),
    "gv_model_mtp_fill": (_c.c_int, [_P, _P, _c.c_int, _c.c_int, _P]),
    "gv_model_set_draft_vocab": (_c.c_int, [_P, _P, _c.c_int]),
    "gv_model_hidden": (_c.c_int, [_P, _P, _c.c_int]),
    "gv_model_draft_logits": (_c.c_int, [_P, _P]),
    "gv_pack_open": (_P, [_c.c_char_p, _c.c_char_p, _c.c_int]),
    "gv_pack_close": (None, [_P]),
    "gv_pack_print": (_c.c_uint64, [_P]),
    "gv_pack_model_config": (_c.c_int, [_P, _c.c_int, _c.c_int, _c.c_int, _c.POINTER(GvModelConfig)]),
    "gv_pack_tensor": (_c.c_int, [_P, _c.c_char_p, _c.POINTER(GvPackTensorInfo)]),
    "gv_pack_expert": (_c.c_int, [_P, _c.c_int, _c.c_int, _P, _P, _P]),
    "gv_pack_tile8": (_c.c_int, [_P]),
    "gv_q4_untile8": (_c.c_int, [_c.c_int64, _c.c_int64, _P, _P]),
    "gv_model_load_pack": (_c.c_int, [_P, _P]),
    "gv_model_save_state": (_c.c_int, [_P, _c.c_char_p, _c.c_int, _c.POINTER(GvStateInfo)]),
    "gv_model_load_state": (_c.c_int, [_P, _c.c_char_p, _c.POINTER(GvStateInfo)]),
    "gv_sample_rows": (_c.c_int, [_P, _c.c_int64, _c.c_int, _c.c_int, _c.c_float, _c.c_float, _c.c_int, _c.c_int,
                                  _P, _P]),
    "gv_accept_match": (_c.c_int, [_P, _c.c_int64, _c.c_int, _P, _c.c_int, _c.c_float, _c.c_float, _c.c_int,
                                   _c.c_int, _P, _P, _P]),
    "gv_accept_match_ex": (_c.c_int, [_P, _c.c_int64, _c.c_int, _P, _c.c_int, _c.c_float, _c.c_float, _c.c_int,
                                      _c.c_int, _P, _P, _c.c_int, _c.c_float, _P, _c.c_int, _P, _P]),
    "gv_sampler_paths": (_c.c_int, [_P, _P]),
    "gv_accept_textbook": (_c.c_int, [_P, _P, _c.c_int64, _c.c_int, _c.c_int, _c.c_float, _c.c_float, _c.c_int,
                                      _P, _P, _c.c_float, _P]),
}

# kernel classes of a verify step (gv_model_time_kernel)
KERNEL_CLASSES = ["embed", "quantize", "qkv", "rope_kv", "attention", "attn_merge", "o_proj", "router", "route",
                  "moe_up", "swiglu", "moe_down", "combine", "lm_head", "gdn_ab", "gdn_conv", "gdn_core", "gdn_norm"]


class GeodeError(RuntimeError):
    pass


# the error classes of gv_model_save_state / gv_model_load_state (GEODE_E_IO, _FORMAT, _ARG, _MEMORY of the
# reference's geode_state_save / geode_state_load)
STATE_ERRORS = {-1: "io", -2: "format", -3: "arg", -4: "memory"}


class StateError(GeodeError):
    """a refused save or load; .kind is one of STATE_ERRORS' values"""

    def __init__(self, kind, msg):
        super().__init__(msg)
        self.kind = kind


def _load():
    if not os.path.exists(LIB_PATH):
        raise GeodeError(f"{LIB_PATH} is not built: run `python -m geode_amd.build` (no CPU fallback exists)")
    lib = _c.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_LIB = None


def _lib():
    """the loaded library (on first use: importing this package, e.g. for geode_amd.build, loads nothing)"""
    global _LIB
    if _LIB is None:
        _LIB = _load()
    return _LIB


def __getattr__(name):   # geode_amd.lib
    if name == "lib":
        return _lib()
    raise AttributeError(name)


def check(rc, what=""):
    if rc != 0:
        raise GeodeError(f"{what}: {_lib().gv_last_error().decode()}")


def init(device=0):
    check(_lib().gv_init(device), "gv_init")


class DeviceBuffer:
    """Device memory owned from Python (gv_malloc / gv_free)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = _lib().gv_malloc(max(1, self.nbytes))
        if not self.ptr:
            raise GeodeError(f"gv_malloc({nbytes}): {_lib().gv_last_error().decode()}")

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(_lib().gv_memcpy_h2d(_c.c_void_p(self.ptr + offset), a.ctypes.data_as(_P), a.nbytes), "h2d")

    def download(self, dtype, shape, offset=0):
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(_lib().gv_memcpy_d2h(out.ctypes.data_as(_P), _c.c_void_p(self.ptr + offset), out.nbytes), "d2h")
        return out

    def zero(self):
        check(_lib().gv_memset(self.ptr, 0, self.nbytes), "memset")

    def __int__(self):
        return self.ptr

    def free(self):
        if self.ptr:
            _lib().gv_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Q4Matrix:
    """A q4 matrix resident on the device in the kernels' layout (from pack-layout bytes)."""

    def __init__(self, pack_bytes, rows, cols, global_):
        pack = np.ascontiguousarray(pack_bytes, np.uint8).reshape(rows, cols // 16 * 9)
        staging = DeviceBuffer.from_array(pack)
        self.buf = DeviceBuffer(_lib().gv_q4_device_bytes(rows, cols))
        self.desc = GvQ4()
        check(_lib().gv_q4_from_pack(staging.ptr, rows, cols, global_, self.buf.ptr, _c.byref(self.desc)),
              "gv_q4_from_pack")
        check(_lib().gv_synchronize(), "sync")
        staging.free()
        self.rows, self.cols = rows, cols

    def ref(self):
        return _c.byref(self.desc)

    def dequant(self):
        out = DeviceBuffer(self.rows * self.cols * 4)
        check(_lib().gv_q4_dequant(self.ref(), out.ptr), "gv_q4_dequant")
        return out.download(np.float32, (self.rows, self.cols))


def act_bytes(cols):
    return _lib().gv_act_bytes(cols)


def gemv(w: Q4Matrix, x: np.ndarray, accumulate_into=None):
    """y = W x for x [M, cols] fp32 (host), on the int8 path; returns y [M, rows]."""
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0]
    dx = DeviceBuffer.from_array(x)
    act = DeviceBuffer(M * act_bytes(w.cols))
    check(_lib().gv_quantize(dx.ptr, w.cols, M, w.cols, None, 0.0, act.ptr, None), "gv_quantize")
    y = DeviceBuffer(M * w.rows * 4)
    if accumulate_into is not None:
        y.upload(np.ascontiguousarray(accumulate_into, np.float32))
    check(_lib().gv_gemv_q4(w.ref(), act.ptr, M, y.ptr, w.rows, int(accumulate_into is not None)), "gv_gemv_q4")
    return y.download(np.float32, (M, w.rows))


def _dev_rows(x):
    """(device buffer or pointer, ld) of a float32 [rows][V] array (uploaded) or an existing device pointer"""
    if isinstance(x, np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        buf = DeviceBuffer.from_array(x)
        return buf, buf.ptr, x.shape[-1]
    raise TypeError("expected a float32 [rows][V] numpy array")


def sample_rows(logits, temperature, top_p=1.0, top_k=0, cap=1024, u=None):
    """Sampler::sample of each row (engine/src/sampler.cpp:16-50) on the GPU with injected uniforms u[r]"""
    buf, ptr, V = _dev_rows(logits)
    rows = logits.shape[0]
    uu = np.ascontiguousarray(u if u is not None else np.zeros(rows), np.float64)
    out = np.empty(rows, np.int32)
    check(_lib().gv_sample_rows(ptr, V, rows, V, temperature, top_p, top_k, cap, uu.ctypes.data_as(_P),
                                out.ctypes.data_as(_P)), "gv_sample_rows")
    return out


def accept_match(logits, batch, temperature, top_p=1.0, top_k=0, cap=1024, u=None):
    """sample-and-match over a verified chain (engine/src/geode.cpp:318-374): (emitted tokens, kept rows)"""
    buf, ptr, V = _dev_rows(logits)
    n = logits.shape[0]
    b = np.ascontiguousarray(batch, np.int32)
    uu = np.ascontiguousarray(u if u is not None else np.zeros(n), np.float64)
    out = np.empty(n, np.int32)
    kept = _c.c_int(0)
    rc = _lib().gv_accept_match(ptr, V, V, b.ctypes.data_as(_P), n, temperature, top_p, top_k, cap,
                                uu.ctypes.data_as(_P), out.ctypes.data_as(_P), _c.byref(kept))
    check(-1 if rc < 0 else 0, "gv_accept_match")
    return out[:rc].copy(), kept.value


def accept_match_ex(logits, batch, temperature, top_p=1.0, top_k=0, cap=1024, u=None, seen=(), presence_penalty=0.0,
                    stop=()):
    """sample-and-match with the generate loop's presence penalty and stop tokens (engine/src/geode.cpp:236-255,
    :331-350): (emitted tokens, kept rows, the rows' logits after the penalty)"""
    buf, ptr, V = _dev_rows(logits)
    n = logits.shape[0]
    b = np.ascontiguousarray(batch, np.int32)
    uu = np.ascontiguousarray(u if u is not None else np.zeros(n), np.float64)
    sn = np.ascontiguousarray(np.asarray(seen, np.int32).reshape(-1))
    st = np.ascontiguousarray(np.asarray(stop, np.int32).reshape(-1))
    out = np.empty(n, np.int32)
    kept = _c.c_int(0)
    rc = _lib().gv_accept_match_ex(ptr, V, V, b.ctypes.data_as(_P), n, temperature, top_p, top_k, cap,
                                   uu.ctypes.data_as(_P), sn.ctypes.data_as(_P), sn.size, presence_penalty,
                                   st.ctypes.data_as(_P), st.size, out.ctypes.data_as(_P), _c.byref(kept))
    check(-1 if rc < 0 else 0, "gv_accept_match_ex")
    return out[:rc].copy(), kept.value, buf.download(np.float32, (n, V))


def accept_textbook(target, draft, temperature, top_p, greedy, u_draft=None, u_acc=None, u_res=0.0):
    """the textbook rule (Leviathan et al. 2023, Alg. 1) on the GPU: the emitted tokens"""
    tb, tp, V = _dev_rows(target)
    db, dp, _ = _dev_rows(draft)
    k = draft.shape[0]
    ud = np.ascontiguousarray(u_draft if u_draft is not None else np.zeros(k), np.float32)
    ua = np.ascontiguousarray(u_acc if u_acc is not None else np.zeros(k), np.float32)
    out = np.empty(k + 1, np.int32)
    rc = _lib().gv_accept_textbook(tp, dp, V, V, k, temperature, top_p, 1 if greedy else 0, ud.ctypes.data_as(_P),
                                   ua.ctypes.data_as(_P), float(u_res), out.ctypes.data_as(_P))
    check(-1 if rc < 0 else 0, "gv_accept_textbook")
    return out[:rc].copy()


def sampler_paths():
    """(sampling calls of the acceptance rules the candidate path decided, calls that ran the full walks) since the
    library loaded"""
    a, b = _c.c_int64(0), _c.c_int64(0)
    check(_lib().gv_sampler_paths(_c.byref(a), _c.byref(b)), "gv_sampler_paths")
    return a.value, b.value


class Pack:
    """A geode-pack opened on the host (Pack::open, engine/src/pack.cpp:39-308): the manifest and its tables checked,
    nothing read until a model loads it."""

    DTYPES = {0: "f32", 1: "bf16", 2: "q2", 3: "q3", 4: "nvfp4", 5: "q8", 6: "q4", 8: "q4i"}

    def __init__(self, directory):
        err = _c.create_string_buffer(512)
        self.h = _lib().gv_pack_open(os.fsencode(directory), err, 512)
        if not self.h:
            raise GeodeError(err.value.decode())

    def close(self):
        if getattr(self, "h", None):
            _lib().gv_pack_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def print(self):
        """FNV-1a of geode.json (the pack print a state file carries)"""
        return _lib().gv_pack_print(self.h)

    @property
    def tile8(self):
        return bool(_lib().gv_pack_tile8(self.h))

    def model_config(self, max_ctx, max_rows=17, kv_int8=0):
        c = GvModelConfig()
        check(_lib().gv_pack_model_config(self.h, max_ctx, max_rows, kv_int8, _c.byref(c)), "gv_pack_model_config")
        return c.to_dict()

    def tensor(self, name):
        t = GvPackTensorInfo()
        check(_lib().gv_pack_tensor(self.h, name.encode(), _c.byref(t)), "gv_pack_tensor")
        return {"type": self.DTYPES.get(t.type, "?"), "rows": t.rows, "cols": t.cols, "file": t.file,
                "offset": t.offset, "bytes": t.bytes, "global": t.global_}

    def expert(self, layer, e):
        f, o, t = _c.c_int(0), _c.c_uint64(0), _c.c_int(0)
        check(_lib().gv_pack_expert(self.h, layer, e, _c.byref(f), _c.byref(o), _c.byref(t)), "gv_pack_expert")
        return f.value, o.value, self.DTYPES.get(t.value, "?")


def q4_untile8(rows, cols, tiled):
    """gv_q4_untile8: tile8 bytes (engine/src/kernels.cpp:971-991) back to the pack's rows"""
    src = np.ascontiguousarray(tiled, np.uint8)
    dst = np.empty_like(src)
    check(_lib().gv_q4_untile8(rows, cols, src.ctypes.data_as(_P), dst.ctypes.data_as(_P)), "gv_q4_untile8")
    return dst


class VerifyModel:
    """A whole model on the device and the verify contract: verify(tokens, parents) then keep(kept, path), as
    Model::verify_n / verify_keep (engine/src/model.cpp:1483-1634)."""

    def __init__(self, cfg: dict):
        self.cfg = dict(cfg)
        c = GvModelConfig.of(cfg)
        err = _c.create_string_buffer(512)
        self.h = _lib().gv_model_create(_c.byref(c), err, 512)
        if not self.h:
            raise GeodeError(f"gv_model_create: {err.value.decode()}")

    def close(self):
        if getattr(self, "h", None):
            _lib().gv_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def adopt(self, kind, data, layer=0, expert=0, globals_=None):
        data = np.ascontiguousarray(data)
        g = np.ascontiguousarray(globals_ if globals_ is not None else [0.0], np.float32)
        check(_lib().gv_model_adopt(self.h, kind, layer, expert, data.ctypes.data_as(_P), data.nbytes,
                                 g.ctypes.data_as(_P)), f"gv_model_adopt({kind}, {layer}, {expert})")

    def randomize(self, seed, sigma=0.02, router_sigma=0.0221, ctx=0):
        check(_lib().gv_model_randomize(self.h, seed, sigma, router_sigma, ctx), "gv_model_randomize")

    @property
    def position(self):
        return _lib().gv_model_position(self.h)

    @position.setter
    def position(self, p):
        check(_lib().gv_model_set_position(self.h, p), "gv_model_set_position")

    def verify(self, tokens, parents=None, want_logits=True):
        tokens = np.ascontiguousarray(tokens, np.int32)
        n = tokens.size
        par = np.ascontiguousarray(parents, np.int32) if parents is not None else None
        out = np.empty((n, self.cfg["vocab"]), np.float32) if want_logits else None
        check(_lib().gv_verify(self.h, tokens.ctypes.data_as(_P), n, par.ctypes.data_as(_P) if par is not None else None,
                            out.ctypes.data_as(_P) if out is not None else None), "gv_verify")
        return out

    def keep(self, kept, path=None):
        p = np.ascontiguousarray(path, np.int32) if path is not None else None
        check(_lib().gv_verify_keep(self.h, kept, p.ctypes.data_as(_P) if p is not None else None), "gv_verify_keep")

    def gdn_state(self, layer):
        """a Gated DeltaNet layer's states as the last verify / keep left them: (conv [2 kd + vd][K - 1],
        S [nv][dk][dv])"""
        c = self.cfg
        conv = np.empty((2 * c["gdn_k_heads"] * c["gdn_k_dim"] + c["gdn_v_heads"] * c["gdn_v_dim"],
                         c["conv_kernel"] - 1), np.float32)
        S = np.empty((c["gdn_v_heads"], c["gdn_k_dim"], c["gdn_v_dim"]), np.float32)
        check(_lib().gv_model_gdn_state(self.h, layer, conv.ctypes.data_as(_P), S.ctypes.data_as(_P)),
              "gv_model_gdn_state")
        return conv, S

    # ---- the MTP draft layer (a model made with mtp = 1)
    @staticmethod
    def _hid(hidden):
        return np.ascontiguousarray(hidden, np.float32) if hidden is not None else None

    def draft(self, tokens, pos, hidden=None):
        """gv_model_draft: (draft token, its probability); hidden None = the last verify's final-normed rows"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        hid = self._hid(hidden)
        d, p = _c.c_int32(0), _c.c_float(0)
        check(_lib().gv_model_draft(self.h, tokens.ctypes.data_as(_P), tokens.size, pos,
                                    hid.ctypes.data_as(_P) if hid is not None else None, _c.byref(d), _c.byref(p)),
              "gv_model_draft")
        return d.value, p.value

    def draft_next(self, token, pos):
        """gv_model_draft_next: (draft token, its probability) from the last MTP pass's output"""
        d, p = _c.c_int32(0), _c.c_float(0)
        check(_lib().gv_model_draft_next(self.h, int(token), pos, _c.byref(d), _c.byref(p)), "gv_model_draft_next")
        return d.value, p.value

    def draft_chain(self, tokens, pos, kmax, pmin=0.8, hidden=None):
        """gv_model_draft_chain: (drafts, probabilities) by the generate loop's rule"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        hid = self._hid(hidden)
        d = np.zeros(max(1, kmax - 1), np.int32)
        p = np.zeros(max(1, kmax - 1), np.float32)
        cnt = _c.c_int(0)
        check(_lib().gv_model_draft_chain(self.h, tokens.ctypes.data_as(_P), tokens.size, pos,
                                          hid.ctypes.data_as(_P) if hid is not None else None, kmax, pmin,
                                          d.ctypes.data_as(_P), p.ctypes.data_as(_P), _c.byref(cnt)),
              "gv_model_draft_chain")
        return d[:cnt.value].copy(), p[:cnt.value].copy()

    def mtp_fill(self, tokens, pos, hidden=None):
        """gv_model_mtp_fill: the MTP layer's KV of a prompt's rows (no logits)"""
        tokens = np.ascontiguousarray(tokens, np.int32)
        hid = self._hid(hidden)
        check(_lib().gv_model_mtp_fill(self.h, tokens.ctypes.data_as(_P), tokens.size, pos,
                                       hid.ctypes.data_as(_P) if hid is not None else None), "gv_model_mtp_fill")

    def set_draft_vocab(self, ids):
        a = np.ascontiguousarray(ids if ids is not None else [], np.int32)
        check(_lib().gv_model_set_draft_vocab(self.h, a.ctypes.data_as(_P), a.size), "gv_model_set_draft_vocab")

    def hidden(self):
        """the last verify's rows after the final norm [n][hidden]"""
        out = np.empty((self.cfg["max_rows"], self.cfg["hidden"]), np.float32)
        n = _lib().gv_model_hidden(self.h, out.ctypes.data_as(_P), out.shape[0])
        if n < 0:
            check(n, "gv_model_hidden")
        return out[:n].copy()

    def draft_logits(self):
        """the last MTP pass's logits (its last row, over the draft head)"""
        out = np.empty(self.cfg["vocab"], np.float32)
        n = _lib().gv_model_draft_logits(self.h, out.ctypes.data_as(_P))
        if n < 0:
            check(n, "gv_model_draft_logits")
        return out[:n].copy()

    def time_kernel(self, cls):
        """events around every launch of kernel class cls (an index into KERNEL_CLASSES; -1 off) from now on"""
        check(_lib().gv_model_time_kernel(self.h, cls), "gv_model_time_kernel")

    def kernel_time(self):
        """(summed ms, launches) of the timed class since time_kernel"""
        ms, n = _c.c_float(0), _c.c_int(0)
        check(_lib().gv_model_kernel_time(self.h, _c.byref(ms), _c.byref(n)), "gv_model_kernel_time")
        return ms.value, n.value

    def set_graphs(self, on):
        """the verify step as one HIP graph per row count (default) or plain launches"""
        check(_lib().gv_model_set_graphs(self.h, 1 if on else 0), "gv_model_set_graphs")

    def set_fused(self, on):
        """dependent phases chained within one launch where the shapes fit (True / 1, the default: with the rows
        routed by the experts' up launch; 2: routed by the output projection's launch) or one launch a phase (0)"""
        check(_lib().gv_model_set_fused(self.h, int(on)), "gv_model_set_fused")

    def trace(self, on):
        """workgroup clock stamps of the traced kernels on or off (a measurement aid)"""
        check(_lib().gv_model_trace(self.h, 1 if on else 0), "gv_model_trace")

    def trace_read(self):
        """the stamps [kernel class][workgroup][slot] in 10 ns ticks (0: not stamped)"""
        n = len(KERNEL_CLASSES) * 8192 * 8
        out = np.zeros(n, np.uint64)
        k = _lib().gv_model_trace_read(self.h, out.ctypes.data, n)
        if k < 0:
            check(-1, "gv_model_trace_read")
        return out.reshape(len(KERNEL_CLASSES), 8192, 8)

    def replay(self, cls, layer=0, reps=20):
        """mean ms a launch of kernel class cls, launched reps times back to back on the last verify's state, launch i
        on layer (layer + i) mod n_layers"""
        ms = _c.c_float(0)
        check(_lib().gv_model_replay(self.h, cls, layer, reps, _c.byref(ms)), "gv_model_replay")
        return ms.value

    def moe(self, layer, h, router_logits=None):
        """one MoE block on rows h [M][hidden] (C3): (out [M][hidden] without the residual, ids, weights)"""
        h = np.ascontiguousarray(h, np.float32)
        M = h.shape[0]
        K, H = self.cfg["top_k"], self.cfg["hidden"]
        lg = np.ascontiguousarray(router_logits, np.float32) if router_logits is not None else None
        out = np.empty((M, H), np.float32)
        ids = np.empty((M, K), np.int32)
        wts = np.empty((M, K), np.float32)
        check(_lib().gv_model_moe(self.h, layer, h.ctypes.data_as(_P), M, lg.ctypes.data_as(_P) if lg is not None
                                  else None, out.ctypes.data_as(_P), ids.ctypes.data_as(_P), wts.ctypes.data_as(_P)),
              "gv_model_moe")
        return out, ids, wts

    def layer(self, layer, x_in, parents=None):
        """one layer on the residual stream x_in [n][hidden] at the current position: (x after the attention, x after
        the MoE, routed ids [n][top_k]); the position does not move"""
        x_in = np.ascontiguousarray(x_in, np.float32)
        n, H, K = x_in.shape[0], self.cfg["hidden"], self.cfg["top_k"]
        par = np.ascontiguousarray(parents, np.int32) if parents is not None else None
        mid = np.empty((n, H), np.float32)
        out = np.empty((n, H), np.float32)
        ids = np.empty((n, K), np.int32)
        check(_lib().gv_model_layer(self.h, layer, x_in.ctypes.data_as(_P), n,
                                    par.ctypes.data_as(_P) if par is not None else None, mid.ctypes.data_as(_P),
                                    out.ctypes.data_as(_P), ids.ctypes.data_as(_P)), "gv_model_layer")
        return mid, out, ids

    def save_state(self, path, append=False, *, pack_print=0, conv_id=0, extra=0, rope_delta=0, has_mtp=False,
                   has_vision=False, hidden=None):
        """Model::save_state (engine/src/state.cpp:251-371): the conversation to path in the reference's state format;
        append: in place when path holds an earlier state of the same conversation. hidden: [hidden] float32 or None
        (the last hidden state an MTP layer drafts from, kept when has_mtp)."""
        hid = np.ascontiguousarray(hidden, np.float32) if hidden is not None else None
        info = GvStateInfo(pack_print, conv_id, extra, rope_delta, int(has_mtp), int(has_vision),
                           hid.ctypes.data_as(_P) if hid is not None else None, 0)
        rc = _lib().gv_model_save_state(self.h, os.fsencode(path), 1 if append else 0, _c.byref(info))
        if rc != 0:
            raise StateError(STATE_ERRORS.get(rc, "io"), _lib().gv_last_error().decode())

    def load_state(self, path, *, pack_print=0, has_mtp=False, has_vision=False):
        """Model::load_state (engine/src/state.cpp:373-463): the saved conversation replaces this one; returns
        {conv_id, extra, rope_delta, hidden (or None)}. On failure StateError and the position is 0."""
        hid = np.zeros(self.cfg["hidden"], np.float32)
        info = GvStateInfo(pack_print, 0, 0, 0, int(has_mtp), int(has_vision), hid.ctypes.data_as(_P), 0)
        rc = _lib().gv_model_load_state(self.h, os.fsencode(path), _c.byref(info))
        if rc != 0:
            raise StateError(STATE_ERRORS.get(rc, "io"), _lib().gv_last_error().decode())
        return {"conv_id": info.conv_id, "extra": info.extra, "rope_delta": info.rope_delta,
                "hidden": hid if info.has_hidden else None}

    def load_pack(self, pack):
        """gv_model_load_pack: every tensor of an open Pack adopted (Model::bind, engine/src/model.cpp:95-202)"""
        check(_lib().gv_model_load_pack(self.h, pack.h), "gv_model_load_pack")

    def moe_replay(self, reps=20):
        """mean ms of the last moe() block re-run on its device-staged inputs (device work only)"""
        ms = _c.c_float(0)
        check(_lib().gv_model_moe_replay(self.h, reps, _c.byref(ms)), "gv_model_moe_replay")
        return ms.value

    def route_ids(self, n):
        out = np.empty((self.cfg["n_layers"], n, self.cfg["top_k"]), np.int32)
        check(_lib().gv_model_route_ids(self.h, out.ctypes.data_as(_P)), "gv_model_route_ids")
        return out
