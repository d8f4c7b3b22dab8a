// oracle_state.cpp - the reference's conversation state file written and read from the CPU oracle's KV cache.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP path's gv_model_save_state / gv_model_load_state,
// never part of it.
//
// A restatement of Model::save_state / load_state (engine/src/state.cpp:251-463) over the oracle's cache, which is the
// reference's chunked layout with one chunk of max_ctx positions ([K, V][max_ctx][kv_row] a layer, the int8 scales
// [K, V][max_ctx][kv_heads]): the block loops copy a run of rows a (block, K/V, layer) as the reference's do.
// Pinning (tests/test_oracle_state.py): FNV-1a against its published test vectors; every byte of a saved file
// against an independent numpy / struct layout of the format (state.cpp:1-20, :53-67, :192-209); the refusals
// (magic, version, checksum, fingerprint, cut short, interrupted, too long) one planted damage each; an append
// against a whole save of the same state.
#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "oracle.h"

namespace {

constexpr char kMagic[8] = {'G', 'E', 'O', 'D', 'E', 'S', 'T', 'A'};
constexpr uint32_t kVersion = 1;
constexpr int kStateBlock = 256;
constexpr uint64_t kHeaderBytes = 4096;

struct StateHeader {   // state.cpp:53-67
    char magic[8];
    uint32_t version, header_size;
    uint64_t fingerprint, conv_id, gen;
    int32_t position, extra, rope_delta;
    uint32_t n_images, image_cap;
    uint32_t kv_elem, n_attn, kv_heads, kv_row, hidden, has_hidden, block;
    uint64_t conv_n, gdn_n;
    uint64_t fixed_offset, fixed_bytes, kv_offset, block_bytes;
    uint64_t checksum;
};

uint64_t fnv(const void *data, size_t n, uint64_t h = 1469598103934665603ull) {   // state.cpp:71-75
    const auto *p = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}
uint64_t checksum(const StateHeader &h) { return fnv(&h, offsetof(StateHeader, checksum)); }

struct Layout {   // state.cpp:192-209
    uint64_t images, hidden, conv, gdn, trail, fixed_bytes, kv_offset;
};
Layout layout(const StateHeader &h) {
    Layout L{};
    L.images = h.fixed_offset + sizeof(uint64_t);
    L.hidden = L.images + static_cast<uint64_t>(h.image_cap) * 4 * sizeof(int32_t);
    L.conv = L.hidden + static_cast<uint64_t>(h.hidden) * sizeof(float);
    L.gdn = L.conv + h.conv_n * sizeof(float);
    L.trail = L.gdn + h.gdn_n * sizeof(float);
    L.fixed_bytes = L.trail + sizeof(uint64_t) - h.fixed_offset;
    L.kv_offset = (h.fixed_offset + L.fixed_bytes + 4095) / 4096 * 4096;
    return L;
}

struct File {
    std::FILE *f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
    bool write(uint64_t off, const void *p, size_t n) {
        return std::fseek(f, static_cast<long>(off), SEEK_SET) == 0 && std::fwrite(p, 1, n, f) == n;
    }
    bool read(uint64_t off, void *p, size_t n) {
        return std::fseek(f, static_cast<long>(off), SEEK_SET) == 0 && std::fread(p, 1, n, f) == n;
    }
    uint64_t size() {
        std::fseek(f, 0, SEEK_END);
        const long n = std::ftell(f);
        return n < 0 ? 0 : static_cast<uint64_t>(n);
    }
};

bool read_header(File &f, StateHeader &h, std::string &err) {   // state.cpp:171-190
    if (!f.read(0, &h, sizeof h)) return err = "not a saved conversation (too short)", false;
    if (std::memcmp(h.magic, kMagic, sizeof kMagic) != 0) return err = "not a saved conversation", false;
    if (h.version != kVersion || h.header_size != sizeof(StateHeader))
        return err = "a saved conversation of another version (" + std::to_string(h.version) + ")", false;
    if (h.checksum != checksum(h)) return err = "the saved conversation's header is damaged", false;
    return true;
}

// the oracle model's view as the reference's Model sees it for a state: the attention layers' KV (n_attn of them, in
// layer order), the Gated DeltaNet layers' states (model.cpp:663-664: conv_n, gdn_n over the GDN layers in order)
struct View {
    orc_config c{};
    size_t elem = 2, kv_row = 0, row_bytes = 0, scale_bytes = 0;
    int n_attn = 0;
    std::vector<uint8_t *> kv;    // [attention layer] rows [K, V][max_ctx][kv_row]
    std::vector<float *> scales;  // [attention layer] int8: [K, V][max_ctx][kv_heads]
    std::vector<float *> conv, S; // [GDN layer] [conv_dim][K - 1], [nv][dk][dv]
    size_t conv_per = 0, s_per = 0;   // floats a GDN layer's conv / recurrent state
    uint64_t conv_n = 0, gdn_n = 0;
};
View view_of(orc_model *m) {
    View v;
    v.c = *orc_model_config(m);
    v.elem = v.c.kv_int8 ? 1 : 2;
    v.kv_row = static_cast<size_t>(v.c.n_kv_heads) * v.c.head_dim;
    v.row_bytes = v.kv_row * v.elem;
    v.scale_bytes = v.c.kv_int8 ? static_cast<size_t>(v.c.n_kv_heads) * sizeof(float) : 0;
    const auto &c = v.c;
    v.conv_per = static_cast<size_t>(2 * c.gdn_k_heads * c.gdn_k_dim + c.gdn_v_heads * c.gdn_v_dim) *
                 static_cast<size_t>(c.conv_kernel > 0 ? c.conv_kernel - 1 : 0);
    v.s_per = static_cast<size_t>(c.gdn_v_heads) * c.gdn_k_dim * c.gdn_v_dim;
    // (the MTP layer's KV after the main layers', model.cpp:351)
    for (int l = 0; l < v.c.n_layers + (c.mtp ? 1 : 0); ++l) {
        int64_t bytes = 0;
        if (c.gdn_v_heads > 0 && l < c.n_layers && c.gdn_layers[l]) {
            v.conv.push_back(reinterpret_cast<float *>(orc_model_tensor(m, ORC_GDN_CONV_ST, l, 0, &bytes, nullptr)));
            v.S.push_back(reinterpret_cast<float *>(orc_model_tensor(m, ORC_GDN_S, l, 0, &bytes, nullptr)));
            continue;
        }
        ++v.n_attn;
        v.kv.push_back(orc_model_tensor(m, v.c.kv_int8 ? ORC_KV8 : ORC_KV, l, 0, &bytes, nullptr));
        v.scales.push_back(v.c.kv_int8 ? reinterpret_cast<float *>(orc_model_tensor(m, ORC_KVS, l, 0, &bytes, nullptr))
                                       : nullptr);
    }
    v.conv_n = v.conv.size() * v.conv_per;
    v.gdn_n = v.S.size() * v.s_per;
    return v;
}

// a head's recurrent state as the reference keeps it (model.cpp:3649-3656): strips of 16 columns, [dv / 16][dk][16]
// (dv a multiple of 16; else [dk][dv] as it is); `to_strips` from [dk][dv] to that, else back
void strips(const float *src, float *dst, int dk, int dv, bool to_strips) {
    if (dv % 16) {
        std::memcpy(dst, src, static_cast<size_t>(dk) * dv * sizeof(float));
        return;
    }
    for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) {
            const size_t rows = static_cast<size_t>(i) * dv + j, strip = (static_cast<size_t>(j / 16) * dk + i) * 16 + j % 16;
            if (to_strips) dst[strip] = src[rows];
            else dst[rows] = src[strip];
        }
}
// every GDN layer's states in the file's order (conv states of each layer, then recurrent states of each layer, in
// strips), or back from it
void gdn_states(const View &v, std::vector<float> &conv, std::vector<float> &gdn, bool to_file) {
    const int nv = v.c.gdn_v_heads, dk = v.c.gdn_k_dim, dv = v.c.gdn_v_dim;
    conv.resize(v.conv_n);
    gdn.resize(v.gdn_n);
    for (size_t g = 0; g < v.conv.size(); ++g) {
        float *fc = conv.data() + g * v.conv_per, *fs = gdn.data() + g * v.s_per;
        if (to_file) std::memcpy(fc, v.conv[g], v.conv_per * sizeof(float));
        else std::memcpy(v.conv[g], fc, v.conv_per * sizeof(float));
        for (int h = 0; h < nv; ++h) {
            const size_t o = static_cast<size_t>(h) * dk * dv;
            if (to_file) strips(v.S[g] + o, fs + o, dk, dv, true);
            else strips(fs + o, v.S[g] + o, dk, dv, false);
        }
    }
}
uint8_t *row_at(const View &v, int l, int which, int p) {   // Model::kv_row_bytes with one chunk (state.cpp:247-251)
    return v.kv[static_cast<size_t>(l)] + (static_cast<size_t>(which) * v.c.max_ctx + static_cast<size_t>(p)) * v.row_bytes;
}
float *scale_at(const View &v, int l, int which, int p) {
    return v.scales[static_cast<size_t>(l)] +
           (static_cast<size_t>(which) * v.c.max_ctx + static_cast<size_t>(p)) * static_cast<size_t>(v.c.n_kv_heads);
}

uint64_t fingerprint(const View &v, const orc_state_info &info) {   // state.cpp:227-245
    const uint64_t shapes[] = {kVersion, v.elem, static_cast<uint64_t>(v.n_attn), static_cast<uint64_t>(v.c.n_kv_heads),
                               v.kv_row, v.conv_n, v.gdn_n, static_cast<uint64_t>(v.c.hidden),
                               static_cast<uint64_t>(v.c.n_layers), info.has_mtp || v.c.mtp ? 1u : 0u, info.has_vision ? 1u : 0u};
    return fnv(shapes, sizeof shapes, info.pack_print ? info.pack_print : 1);
}

void put(char *err, int err_len, const std::string &e) {
    if (err && err_len > 0) {
        std::strncpy(err, e.c_str(), static_cast<size_t>(err_len) - 1);
        err[err_len - 1] = '\0';
    }
}

}  // namespace

extern "C" {

uint64_t orc_fnv1a(const void *data, size_t n, uint64_t seed) { return fnv(data, n, seed); }

int orc_state_save(orc_model *m, const char *path, int append, const orc_state_info *info, char *err, int err_len) {
    const View v = view_of(m);
    const int pos = orc_model_position(m);
    StateHeader h{};
    std::memcpy(h.magic, kMagic, sizeof kMagic);
    h.version = kVersion;
    h.header_size = sizeof(StateHeader);
    h.fingerprint = fingerprint(v, *info);
    h.conv_id = info->conv_id;
    h.gen = 1;
    h.position = pos;
    h.extra = info->extra;
    h.rope_delta = info->rope_delta;
    h.n_images = 0;
    h.image_cap = 16;   // std::max(16, (0 + 15) / 16 * 16 + 16) = 16 with no images
    h.kv_elem = static_cast<uint32_t>(v.elem);
    h.n_attn = static_cast<uint32_t>(v.n_attn);
    h.kv_heads = static_cast<uint32_t>(v.c.n_kv_heads);
    h.kv_row = static_cast<uint32_t>(v.kv_row);
    h.hidden = static_cast<uint32_t>(v.c.hidden);
    h.has_hidden = (info->has_mtp || v.c.mtp) && pos > 0 && info->hidden ? 1 : 0;
    h.block = kStateBlock;
    h.conv_n = v.conv_n;
    h.gdn_n = v.gdn_n;
    h.fixed_offset = kHeaderBytes;
    h.block_bytes = 2 * static_cast<uint64_t>(v.n_attn) * kStateBlock * (v.row_bytes + v.scale_bytes);
    int first_block = 0;
    bool in_place = false;
    if (append) {   // state.cpp:283-299
        File f;
        f.f = std::fopen(path, "rb");
        StateHeader old{};
        std::string e;
        if (f.f && read_header(f, old, e) && old.fingerprint == h.fingerprint && old.conv_id == h.conv_id &&
            old.position <= h.position && h.n_images <= old.image_cap && old.block == h.block &&
            old.block_bytes == h.block_bytes && old.fixed_offset == h.fixed_offset) {
            h.image_cap = old.image_cap;
            h.gen = old.gen + 1;
            first_block = std::max(0, old.position - 1) / kStateBlock;
            in_place = true;
        }
    }
    const Layout L = layout(h);
    h.fixed_bytes = L.fixed_bytes;
    h.kv_offset = L.kv_offset;
    h.checksum = checksum(h);
    const std::string target = in_place ? std::string(path) : std::string(path) + ".tmp";
    File f;
    f.f = std::fopen(target.c_str(), in_place ? "r+b" : "w+b");
    if (!f.f) return put(err, err_len, "cannot write " + target), -1;
    {
        std::vector<uint8_t> head(static_cast<size_t>(L.conv - h.fixed_offset), 0);
        std::memcpy(head.data(), &h.gen, sizeof h.gen);
        if (h.has_hidden) std::memcpy(head.data() + (L.hidden - h.fixed_offset), info->hidden, h.hidden * sizeof(float));
        std::vector<float> conv, gdn;
        gdn_states(v, conv, gdn, true);
        if (!f.write(h.fixed_offset, head.data(), head.size()) || !f.write(L.conv, conv.data(), conv.size() * sizeof(float)) ||
            !f.write(L.gdn, gdn.data(), gdn.size() * sizeof(float)) || !f.write(L.trail, &h.gen, sizeof h.gen))
            return put(err, err_len, "cannot write the states"), -1;
    }
    const int blocks = (pos + kStateBlock - 1) / kStateBlock;
    std::vector<uint8_t> blk(static_cast<size_t>(h.block_bytes));
    for (int b = first_block; b < blocks; ++b) {   // state.cpp:333-358, a block a write
        std::fill(blk.begin(), blk.end(), uint8_t{0});
        const int p0 = b * kStateBlock, p1 = std::min(pos, p0 + kStateBlock);
        uint8_t *scales = blk.data() + 2 * static_cast<size_t>(v.n_attn) * kStateBlock * v.row_bytes;
        for (int which = 0; which < 2; ++which)
            for (int l = 0; l < v.n_attn; ++l) {
                const size_t seg = static_cast<size_t>(which * v.n_attn + l) * kStateBlock;
                std::memcpy(blk.data() + seg * v.row_bytes, row_at(v, l, which, p0), static_cast<size_t>(p1 - p0) * v.row_bytes);
                if (v.scale_bytes)
                    std::memcpy(scales + seg * v.scale_bytes, scale_at(v, l, which, p0),
                                static_cast<size_t>(p1 - p0) * v.scale_bytes);
            }
        if (!f.write(h.kv_offset + static_cast<uint64_t>(b) * h.block_bytes, blk.data(), blk.size()))
            return put(err, err_len, "cannot write the KV cache"), -1;
    }
    if (!f.write(0, &h, sizeof h)) return put(err, err_len, "cannot write the header"), -1;
    std::fclose(f.f);
    f.f = nullptr;
    if (!in_place && std::rename(target.c_str(), path) != 0) return put(err, err_len, "cannot move " + target), -1;
    return 0;
}

int orc_state_load(orc_model *m, const char *path, orc_state_info *info, char *err, int err_len) {
    const View v = view_of(m);
    auto reset = [&] {   // Model::reset (model.cpp:1918-1925): an empty conversation, the GDN states zero
        orc_model_set_position(m, 0);
        info->has_hidden = 0;
        for (float *c : v.conv) std::fill(c, c + v.conv_per, 0.0f);
        for (float *st : v.S) std::fill(st, st + v.s_per, 0.0f);
    };
    reset();
    auto refuse = [&](const std::string &e) {
        reset();
        put(err, err_len, e);
        return -1;
    };
    File f;
    f.f = std::fopen(path, "rb");
    if (!f.f) return refuse(std::string("cannot open ") + path);
    StateHeader h{};
    std::string e;
    if (!read_header(f, h, e)) return refuse(e);
    if (h.fingerprint != fingerprint(v, *info) || h.kv_elem != v.elem || h.n_attn != static_cast<uint32_t>(v.n_attn) ||
        h.kv_heads != static_cast<uint32_t>(v.c.n_kv_heads) || h.kv_row != v.kv_row ||
        h.hidden != static_cast<uint32_t>(v.c.hidden) || h.conv_n != v.conv_n || h.gdn_n != v.gdn_n || h.block == 0)
        return refuse("the conversation was saved by another model or another KV cache format");
    if (h.position < 0 || h.position >= v.c.max_ctx)
        return refuse("the saved conversation (" + std::to_string(h.position) + " tokens) is longer than this context");
    const Layout L = layout(h);
    const int B = static_cast<int>(h.block);
    const int blocks = (h.position + B - 1) / B;
    if (L.fixed_bytes != h.fixed_bytes || L.kv_offset != h.kv_offset || h.n_images > h.image_cap ||
        h.block_bytes != 2 * static_cast<uint64_t>(v.n_attn) * static_cast<uint64_t>(B) * (v.row_bytes + v.scale_bytes) ||
        f.size() < h.kv_offset + static_cast<uint64_t>(blocks) * h.block_bytes)
        return refuse("the saved conversation is cut short");
    uint64_t lead = 0, trail = 0;
    if (!f.read(h.fixed_offset, &lead, sizeof lead) || !f.read(L.trail, &trail, sizeof trail) || lead != h.gen ||
        trail != h.gen)
        return refuse("the saved conversation is incomplete (its save was interrupted)");
    if (h.n_images != 0) return refuse("the saved conversation holds images");
    if (h.has_hidden && info->hidden) {
        if (!f.read(L.hidden, info->hidden, h.hidden * sizeof(float))) return refuse("cannot read the last state");
        info->has_hidden = 1;
    }
    {
        std::vector<float> conv(v.conv_n), gdn(v.gdn_n);
        if (!f.read(L.conv, conv.data(), conv.size() * sizeof(float)) || !f.read(L.gdn, gdn.data(), gdn.size() * sizeof(float)))
            return refuse("cannot read the states");
        gdn_states(v, conv, gdn, false);
    }
    std::vector<uint8_t> blk(static_cast<size_t>(h.block_bytes));
    for (int b = 0; b < blocks; ++b) {   // state.cpp:428-455 (any block size)
        if (!f.read(h.kv_offset + static_cast<uint64_t>(b) * h.block_bytes, blk.data(), blk.size()))
            return refuse("cannot read the KV cache");
        const int p0 = b * B, p1 = std::min(h.position, p0 + B);
        const uint8_t *scales = blk.data() + 2 * static_cast<size_t>(v.n_attn) * static_cast<size_t>(B) * v.row_bytes;
        for (int which = 0; which < 2; ++which)
            for (int l = 0; l < v.n_attn; ++l) {
                const size_t seg = static_cast<size_t>(which * v.n_attn + l) * static_cast<size_t>(B);
                std::memcpy(row_at(v, l, which, p0), blk.data() + seg * v.row_bytes, static_cast<size_t>(p1 - p0) * v.row_bytes);
                if (v.scale_bytes)
                    std::memcpy(scale_at(v, l, which, p0), scales + seg * v.scale_bytes,
                                static_cast<size_t>(p1 - p0) * v.scale_bytes);
            }
    }
    orc_model_set_position(m, h.position);
    info->conv_id = h.conv_id;
    info->extra = h.extra;
    info->rope_delta = h.rope_delta;
    return 0;
}

}  // extern "C"
