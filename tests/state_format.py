"""The reference's conversation state file (engine/src/state.cpp:1-20, the header :53-67, the fixed part's layout
:192-209, the blocks :333-358), restated with struct and numpy for the tests: it writes the bytes a save must
produce from a KV cache given as the reference's rows, and reads a file's parts back. Independent of both the oracle's
C++ and the HIP library's code, so that a mistake in either shows as a byte difference."""
import struct

import numpy as np

MAGIC = b"GEODESTA"
VERSION = 1
BLOCK = 256
HEADER_BYTES = 4096
# magic, version, header_size, fingerprint, conv_id, gen, position, extra, rope_delta, n_images, image_cap, kv_elem,
# n_attn, kv_heads, kv_row, hidden, has_hidden, block, conv_n, gdn_n, fixed_offset, fixed_bytes, kv_offset,
# block_bytes, checksum
HEADER = struct.Struct("<8sIIQQQiiiIIIIIIIIIQQQQQQQ")
FIELDS = ("magic", "version", "header_size", "fingerprint", "conv_id", "gen", "position", "extra", "rope_delta",
          "n_images", "image_cap", "kv_elem", "n_attn", "kv_heads", "kv_row", "hidden", "has_hidden", "block",
          "conv_n", "gdn_n", "fixed_offset", "fixed_bytes", "kv_offset", "block_bytes", "checksum")
M64 = (1 << 64) - 1
# the reference's FNV-1a starts from 1469598103934665603 (state.cpp:68), the first 19 of the 20 digits of FNV's
# published 64-bit offset basis 14695981039346656037; its files carry checksums and fingerprints from that start
REF_BASIS = 1469598103934665603
FNV_BASIS = 14695981039346656037


def fnv1a(data: bytes, h=REF_BASIS):
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & M64
    return h


def fingerprint(pack_print, kv_elem, n_attn, kv_heads, kv_row, hidden, has_mtp=False, has_vision=False, conv_n=0,
                gdn_n=0, n_layers=None):
    """Model::fingerprint (state.cpp:227-245): the attention layers, the Gated DeltaNet states' sizes, all layers"""
    shapes = np.array([VERSION, kv_elem, n_attn, kv_heads, kv_row, conv_n, gdn_n, hidden,
                       n_attn if n_layers is None else n_layers, int(has_mtp), int(has_vision)], "<u8")
    return fnv1a(shapes.tobytes(), pack_print or 1)


def strips(S):
    """a GDN layer's recurrent state [nv][dk][dv] as the reference keeps it (model.cpp:3649-3656): each head in
    strips of 16 columns, [nv][dv / 16][dk][16] (as it is when dv is not a multiple of 16)"""
    nv, dk, dv = S.shape
    if dv % 16:
        return np.ascontiguousarray(S)
    return np.ascontiguousarray(S.reshape(nv, dk, dv // 16, 16).transpose(0, 2, 1, 3))


def unstrips(flat, nv, dk, dv):
    if dv % 16:
        return flat.reshape(nv, dk, dv)
    return np.ascontiguousarray(flat.reshape(nv, dv // 16, dk, 16).transpose(0, 2, 1, 3).reshape(nv, dk, dv))


def layout(h):
    """where the fixed part's pieces start, its size and the KV blocks' offset"""
    images = h["fixed_offset"] + 8
    hidden = images + h["image_cap"] * 16
    conv = hidden + h["hidden"] * 4
    gdn = conv + h["conv_n"] * 4
    trail = gdn + h["gdn_n"] * 4
    fixed_bytes = trail + 8 - h["fixed_offset"]
    kv_offset = (h["fixed_offset"] + fixed_bytes + 4095) // 4096 * 4096
    return dict(images=images, hidden=hidden, conv=conv, gdn=gdn, trail=trail, fixed_bytes=fixed_bytes,
                kv_offset=kv_offset)


def pack_header(h):
    h = dict(h)
    raw = HEADER.pack(*[h[f] if f != "checksum" else 0 for f in FIELDS])
    h["checksum"] = fnv1a(raw[:-8])
    return HEADER.pack(*[h[f] for f in FIELDS]), h


def read_header(buf: bytes):
    return dict(zip(FIELDS, HEADER.unpack_from(buf, 0)))


def state_bytes(cfg, rows, scales, position, *, pack_print=0, conv_id=0, extra=0, rope_delta=0, gen=1,
                has_mtp=False, has_vision=False, hidden=None, block=BLOCK, gdn=()):
    """The file a whole save writes. rows: per attention layer [2][>= position][kv_row] (uint16 fp16 bits or int8),
    scales: per attention layer [2][>= position][kv_heads] float32 (int8 cache) or None; gdn: per Gated DeltaNet
    layer (conv [conv_dim][K - 1], S [nv][dk][dv]) float32."""
    i8 = bool(cfg.get("kv_int8"))
    kv_row = cfg["n_kv_heads"] * cfg["head_dim"]
    L = len(rows)
    elem = 1 if i8 else 2
    scale_bytes = cfg["n_kv_heads"] * 4 if i8 else 0
    has_hidden = int(bool(has_mtp) and position > 0 and hidden is not None)
    conv = b"".join(np.asarray(c, "<f4").tobytes() for c, _ in gdn)
    rec = b"".join(strips(np.asarray(S, "<f4")).tobytes() for _, S in gdn)
    conv_n, gdn_n = len(conv) // 4, len(rec) // 4
    h = dict(magic=MAGIC, version=VERSION, header_size=HEADER.size,
             fingerprint=fingerprint(pack_print, elem, L, cfg["n_kv_heads"], kv_row, cfg["hidden"], has_mtp, has_vision,
                                     conv_n, gdn_n, cfg["n_layers"]),
             conv_id=conv_id, gen=gen, position=position, extra=extra, rope_delta=rope_delta, n_images=0, image_cap=16,
             kv_elem=elem, n_attn=L, kv_heads=cfg["n_kv_heads"], kv_row=kv_row, hidden=cfg["hidden"],
             has_hidden=has_hidden, block=block, conv_n=conv_n, gdn_n=gdn_n, fixed_offset=HEADER_BYTES, fixed_bytes=0,
             kv_offset=0, block_bytes=2 * L * block * (kv_row * elem + scale_bytes), checksum=0)
    lo = layout(h)
    h["fixed_bytes"], h["kv_offset"] = lo["fixed_bytes"], lo["kv_offset"]
    head, h = pack_header(h)
    blocks = -(-position // block)
    # the file ends with the last block written, or with the fixed part when there is none
    out = bytearray(lo["kv_offset"] + blocks * h["block_bytes"] if blocks else lo["trail"] + 8)
    out[:len(head)] = head
    struct.pack_into("<Q", out, h["fixed_offset"], gen)
    struct.pack_into("<Q", out, lo["trail"], gen)
    if has_hidden:
        out[lo["hidden"]:lo["hidden"] + 4 * cfg["hidden"]] = np.asarray(hidden, "<f4").tobytes()
    out[lo["conv"]:lo["conv"] + len(conv)] = conv
    out[lo["gdn"]:lo["gdn"] + len(rec)] = rec
    dt = np.int8 if i8 else np.dtype("<u2")
    for b in range(blocks):
        p0, p1 = b * block, min(position, (b + 1) * block)
        blk = np.zeros((2, L, block, kv_row), dt)
        sc = np.zeros((2, L, block, cfg["n_kv_heads"]), "<f4")
        for l in range(L):
            blk[:, l, :p1 - p0] = rows[l][:, p0:p1]
            if i8:
                sc[:, l, :p1 - p0] = scales[l][:, p0:p1]
        at = lo["kv_offset"] + b * h["block_bytes"]
        data = blk.tobytes() + (sc.tobytes() if i8 else b"")
        out[at:at + len(data)] = data
    return bytes(out)


def kv_rows(cfg, buf: bytes):
    """the KV rows (per layer [2][position][kv_row]) and scales a file holds"""
    h = read_header(buf)
    lo = layout(h)
    i8 = h["kv_elem"] == 1
    L, B, kv_row, nkv, pos = h["n_attn"], h["block"], h["kv_row"], h["kv_heads"], h["position"]
    dt = np.int8 if i8 else np.dtype("<u2")
    rows = [np.zeros((2, pos, kv_row), dt) for _ in range(L)]
    scales = [np.zeros((2, pos, nkv), "<f4") for _ in range(L)] if i8 else None
    for b in range(-(-pos // B)):
        at = lo["kv_offset"] + b * h["block_bytes"]
        nrow = 2 * L * B * kv_row
        blk = np.frombuffer(buf, dt, nrow, at).reshape(2, L, B, kv_row)
        p0, p1 = b * B, min(pos, (b + 1) * B)
        for l in range(L):
            rows[l][:, p0:p1] = blk[:, l, :p1 - p0]
        if i8:
            sc = np.frombuffer(buf, "<f4", 2 * L * B * nkv, at + nrow * np.dtype(dt).itemsize).reshape(2, L, B, nkv)
            for l in range(L):
                scales[l][:, p0:p1] = sc[:, l, :p1 - p0]
    return rows, scales


def gdn_states(cfg, buf: bytes):
    """the Gated DeltaNet layers' states a file holds: per GDN layer (conv [conv_dim][K - 1], S [nv][dk][dv])"""
    h = read_header(buf)
    lo = layout(h)
    n = sum(1 for l in range(cfg["n_layers"]) if cfg.get("gdn_layers") and cfg["gdn_layers"][l])
    if n == 0:
        return []
    nv, dk, dv, K = cfg["gdn_v_heads"], cfg["gdn_k_dim"], cfg["gdn_v_dim"], cfg["conv_kernel"]
    conv_dim = 2 * cfg["gdn_k_heads"] * dk + nv * dv
    cp, sp = conv_dim * (K - 1), nv * dk * dv
    conv = np.frombuffer(buf, "<f4", n * cp, lo["conv"]).reshape(n, conv_dim, K - 1)
    rec = np.frombuffer(buf, "<f4", n * sp, lo["gdn"]).reshape(n, sp)
    return [(conv[g].copy(), unstrips(rec[g], nv, dk, dv)) for g in range(n)]
