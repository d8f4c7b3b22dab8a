// state.hip - a conversation's state in a file and back for the GPU model, in the reference's state format
// (engine/src/state.cpp:1-20, Model::save_state / load_state :251-465), so that a state saved by the reference's CPU
// path loads here and the other way round.
//
// The file (little-endian): [0, 4096) the header, an FNV-1a checksum of its bytes last; at fixed_offset the fixed
// part (gen, the images' (kv0, s, gh, gw) x image_cap, the last hidden state, the GDN layers' conv then recurrent
// states, gen again); at kv_offset (4 KB aligned) the KV cache in blocks of 256 positions, [K, V][attention layer]
// [256][kv_row] elements, then for an int8 cache the scales [K, V][attention layer][256][kv_heads] floats; positions
// past the conversation's end are zeros. The Gated DeltaNet layers' states are those of the model's base slot: each
// layer's conv state [conv_dim][K - 1], then each layer's recurrent state with each head in the reference's strips of
// 16 columns ([dv / 16][dk][16], model.cpp:3649-3656). The model takes no images: the image table is zeros.
//
// Device side: one kernel converts a run of whole blocks between the cache's device layout (K [nkv][slots][hd],
// V [nkv][slots / 64][hd][64], the int8 scales [K, V][nkv][slots]) and the file's, every attention layer at once; the
// host moves batches of up to 16 MB of blocks between a device buffer and the file.
#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "layer_common.hpp"
#include "model.hpp"

namespace gv {
namespace {

constexpr char kMagic[8] = {'G', 'E', 'O', 'D', 'E', 'S', 'T', 'A'};
constexpr uint32_t kVersion = 1;
constexpr int kStateBlock = 256;                 // positions a KV block of the file holds
constexpr uint64_t kHeaderBytes = 4096;
constexpr size_t kIoBatch = size_t{16} << 20;    // the blocks converted and moved at once

// the header's fields in the format's order and sizes (state.cpp:53-67)
struct StateHeader {
    char magic[8];
    uint32_t version, header_size;
    uint64_t fingerprint;
    uint64_t conv_id;
    uint64_t gen;
    int32_t position;
    int32_t extra;
    int32_t rope_delta;
    uint32_t n_images, image_cap;
    uint32_t kv_elem, n_attn, kv_heads, kv_row, hidden, has_hidden, block;
    uint64_t conv_n, gdn_n;
    uint64_t fixed_offset, fixed_bytes, kv_offset, block_bytes;
    uint64_t checksum;   // FNV-1a 64 of every byte before it
};
static_assert(sizeof(StateHeader) == 144 && offsetof(StateHeader, checksum) == 136, "the format's header layout");

uint64_t fnv(const void *data, size_t n, uint64_t h = 1469598103934665603ull) {
    const auto *p = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}
uint64_t header_checksum(const StateHeader &h) { return fnv(&h, offsetof(StateHeader, checksum)); }
uint64_t align4k(uint64_t x) { return (x + 4095) / 4096 * 4096; }

// where the fixed part's pieces are (state.cpp:192-209)
struct Layout {
    uint64_t images, hidden, conv, gdn, trail, fixed_bytes, kv_offset;
};
Layout layout_of(const StateHeader &h) {
    Layout L{};
    L.images = h.fixed_offset + 8;
    L.hidden = L.images + static_cast<uint64_t>(h.image_cap) * 16;
    L.conv = L.hidden + static_cast<uint64_t>(h.hidden) * 4;
    L.gdn = L.conv + h.conv_n * 4;
    L.trail = L.gdn + h.gdn_n * 4;
    L.fixed_bytes = L.trail + 8 - h.fixed_offset;
    L.kv_offset = align4k(h.fixed_offset + L.fixed_bytes);
    return L;
}

struct Shapes {
    uint32_t elem, kv_row, scale_bytes;   // a position's element size, row length and (int8) scale bytes
    uint64_t block_bytes;
};
Shapes shapes_of(const Model &m) {
    Shapes s{};
    s.elem = m.kv_i8 ? 1 : 2;
    s.kv_row = static_cast<uint32_t>(m.c.n_kv_heads * m.c.head_dim);
    s.scale_bytes = m.kv_i8 ? static_cast<uint32_t>(m.c.n_kv_heads) * 4 : 0;
    s.block_bytes = 2 * static_cast<uint64_t>(m.attn_layers.size()) * kStateBlock * (uint64_t{s.kv_row} * s.elem + s.scale_bytes);
    return s;
}
uint64_t conv_n_of(const Model &m) { return m.gdn_layers.size() * static_cast<uint64_t>(gdn_c_floats(m.c)); }
uint64_t gdn_n_of(const Model &m) { return m.gdn_layers.size() * static_cast<uint64_t>(gdn_s_floats(m.c)); }

// Model::fingerprint (state.cpp:227-245): the pack's print folded with the shapes a state holds
uint64_t fingerprint_of(const Model &m, const gv_state_info &info) {
    const auto &c = m.c;
    const uint64_t shapes[] = {kVersion,
                               m.kv_i8 ? 1u : 2u,
                               static_cast<uint64_t>(m.attn_layers.size()),
                               static_cast<uint64_t>(c.n_kv_heads),
                               static_cast<uint64_t>(c.n_kv_heads) * static_cast<uint64_t>(c.head_dim),
                               conv_n_of(m),
                               gdn_n_of(m),
                               static_cast<uint64_t>(c.hidden),
                               static_cast<uint64_t>(c.n_layers),
                               info.has_mtp || m.has_mtp ? 1u : 0u,
                               info.has_vision ? 1u : 0u};
    return fnv(shapes, sizeof shapes, info.pack_print ? info.pack_print : 1);
}

// the Gated DeltaNet layers' states of the base slot in the file's order and layout (conv of every layer, then the
// recurrent state of every layer in strips), or back into the base slot
int gdn_states_io(Model &m, std::vector<float> &conv, std::vector<float> &rec, bool to_file) {
    const auto &c = m.c;
    const int nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim;
    const size_t cp = static_cast<size_t>(gdn_c_floats(c)), sp = static_cast<size_t>(gdn_s_floats(c));
    conv.resize(m.gdn_layers.size() * cp);
    rec.resize(m.gdn_layers.size() * sp);
    std::vector<float> S(sp);
    for (size_t g = 0; g < m.gdn_layers.size(); ++g) {
        LayerW &L = m.layers[static_cast<size_t>(m.gdn_layers[g])];
        float *fc = conv.data() + g * cp, *fs = rec.data() + g * sp;
        if (to_file && gdn_get_state(m, L, m.gdn_base, fc, S.data()) != 0) return -1;
        for (int h = 0; h < nv; ++h)
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j) {   // (dv is a power of two of at least 16: the strips always apply)
                    const size_t o = static_cast<size_t>(h) * dk * dv, rows = o + static_cast<size_t>(i) * dv + j;
                    const size_t strip = o + (static_cast<size_t>(j / 16) * dk + i) * 16 + j % 16;
                    if (to_file) fs[strip] = S[rows];
                    else S[rows] = fs[strip];
                }
        if (!to_file && gdn_put_state(m, L, m.gdn_base, fc, S.data()) != 0) return -1;
    }
    return 0;
}

// Model::reset's states (model.cpp:1918-1925): every Gated DeltaNet slot zero
int gdn_zero(Model &m) {
    const size_t cb = 2 * static_cast<size_t>(m.c.max_rows) * gdn_c_floats(m.c) * 4,
                 sb = 2 * static_cast<size_t>(m.c.max_rows) * gdn_s_floats(m.c) * 4;
    for (int l : m.gdn_layers) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        GV_CHECK_HIP(hipMemsetAsync(L.c_slots, 0, cb, stream()));
        GV_CHECK_HIP(hipMemsetAsync(L.s_slots, 0, sb, stream()));
    }
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    return 0;
}

// Whole blocks [b0, b0 + nb) of B positions between the device cache and the file's layout at `file`, every
// attention layer (n_layers of them, model layer attn_index[l]);
// positions from `position` on are zeros in the file and left alone on the device. A thread per (block, K/V, layer,
// position, 16-byte word of the row), then for an int8 cache a thread per (block, K/V, layer, position) for its
// scales.
template <typename T, bool TO_FILE>
__global__ __launch_bounds__(256) void state_blocks_kernel(uint8_t *kv_all, size_t layer_bytes,
                                                           const int *__restrict__ attn_index, int n_layers, int nkv,
                                                           int hd, int64_t slots, int B, int b0, int nb, int position,
                                                           uint8_t *file) {
    constexpr int E = 16 / sizeof(T);   // elements a word
    constexpr bool kScales = sizeof(T) == 1;
    const int words = nkv * hd / E;
    const int64_t rows = 2 * static_cast<int64_t>(n_layers) * B;   // (K/V, layer, position) of a block
    const int64_t row_bytes = static_cast<int64_t>(nkv) * hd * sizeof(T);
    const int64_t block_bytes = rows * (row_bytes + (kScales ? nkv * 4 : 0));
    const int64_t per_block = rows * (words + (kScales ? 1 : 0));
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= per_block * nb) return;
    const int bi = static_cast<int>(i / per_block);
    int64_t r = i % per_block;
    uint8_t *blk = file + bi * block_bytes;
    const bool scale_item = kScales && r >= rows * words;
    if (scale_item) r -= rows * words;
    const int64_t row = scale_item ? r : r / words;   // (v * n_layers + l) * B + q
    const int v = static_cast<int>(row / (static_cast<int64_t>(n_layers) * B));
    const int l = static_cast<int>((row / B) % n_layers), q = static_cast<int>(row % B);
    const int64_t p = static_cast<int64_t>(b0 + bi) * B + q;
    const bool live = p < position;
    T *kv = reinterpret_cast<T *>(kv_all + static_cast<size_t>(attn_index[l]) * layer_bytes);
    if (scale_item) {
        float *fs = reinterpret_cast<float *>(blk + rows * row_bytes) + row * nkv;
        float *sc = reinterpret_cast<float *>(kv + 2 * static_cast<int64_t>(nkv) * slots * hd);
        for (int kh = 0; kh < nkv; ++kh) {
            if (TO_FILE) fs[kh] = live ? sc[kv_scale_index(slots, nkv, v, kh, p)] : 0.0f;
            else if (live) sc[kv_scale_index(slots, nkv, v, kh, p)] = fs[kh];
        }
        return;
    }
    const int e0 = static_cast<int>(r % words) * E, kh = e0 / hd, d0 = e0 % hd;
    T *fw = reinterpret_cast<T *>(blk + row * row_bytes) + e0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (!live) {
            if (TO_FILE) fw[e] = T(0);
            continue;
        }
        const int64_t at = v == 0 ? k_index(slots, hd, kh, p, d0 + e) : v_index(slots, hd, nkv, kh, p, d0 + e);
        if (TO_FILE) fw[e] = kv[at];
        else kv[at] = fw[e];
    }
}

template <bool TO_FILE>
void launch_blocks(Model &m, int B, int b0, int nb, int position, uint8_t *dev_file, hipStream_t st) {
    const auto &c = m.c;
    const int E = m.kv_i8 ? 16 : 8;
    const int n_attn = static_cast<int>(m.attn_layers.size());
    const int64_t per_block = 2 * static_cast<int64_t>(n_attn) * B * (c.n_kv_heads * c.head_dim / E + (m.kv_i8 ? 1 : 0));
    if (per_block == 0) return;   // (no attention layer)
    const int64_t n = per_block * nb;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256)), block(256);
    auto *base = reinterpret_cast<uint8_t *>(m.kv_all);
    if (m.kv_i8)
        hipLaunchKernelGGL((state_blocks_kernel<int8_t, TO_FILE>), grid, block, 0, st, base, m.kv_layer_bytes,
                           m.attn_index, n_attn, c.n_kv_heads, c.head_dim, m.slots, B, b0, nb, position, dev_file);
    else
        hipLaunchKernelGGL((state_blocks_kernel<_Float16, TO_FILE>), grid, block, 0, st, base, m.kv_layer_bytes,
                           m.attn_index, n_attn, c.n_kv_heads, c.head_dim, m.slots, B, b0, nb, position, dev_file);
}

// The state file's I/O: positioned transfers (pread / pwrite in pieces of at most 1 GB, resumed after a short one),
// its length, and fsync, which orders a save's parts on the disk (a header is never written ahead of what it names).
class StateIo {
public:
    enum Mode { kRead, kUpdate, kCreate };   // read only; read and write in place; a new file (truncated)
    ~StateIo() { shut(); }
    bool open(const std::string &path, Mode mode) {
        const int how = mode == kRead ? O_RDONLY : mode == kUpdate ? O_RDWR : (O_RDWR | O_CREAT | O_TRUNC);
        fd_ = ::open(path.c_str(), how | O_CLOEXEC, 0600);
        return fd_ >= 0;
    }
    void shut() {
        if (fd_ >= 0) ::close(fd_);
        fd_ = -1;
    }
    uint64_t length() const {
        struct stat st {};
        return fd_ >= 0 && fstat(fd_, &st) == 0 ? static_cast<uint64_t>(st.st_size) : 0;
    }
    bool put(uint64_t at, const void *src, size_t n) { return transfer(at, const_cast<void *>(src), n, true); }
    bool get(uint64_t at, void *dst, size_t n) { return transfer(at, dst, n, false); }
    bool flush() { return fd_ >= 0 && ::fsync(fd_) == 0; }

private:
    bool transfer(uint64_t at, void *buf, size_t n, bool out) {
        auto *p = static_cast<uint8_t *>(buf);
        for (size_t left = n; left > 0;) {
            const size_t piece = std::min<size_t>(left, size_t{1} << 30);
            const ssize_t moved = out ? ::pwrite(fd_, p, piece, static_cast<off_t>(at))
                                      : ::pread(fd_, p, piece, static_cast<off_t>(at));
            if (moved <= 0) return false;
            p += moved;
            at += static_cast<uint64_t>(moved);
            left -= static_cast<size_t>(moved);
        }
        return true;
    }
    int fd_ = -1;
};

// the header read and checked in the order a reader relies on it: present, the format's magic, its version and
// size, then its checksum over every byte before the checksum field
bool read_header(StateIo &f, StateHeader &h, std::string &err) {
    if (!f.get(0, &h, sizeof h)) return err = "the file is shorter than a state header", false;
    if (std::memcmp(h.magic, kMagic, sizeof kMagic) != 0) return err = "the file has no state-file magic", false;
    if (h.version != kVersion || h.header_size != sizeof(StateHeader))
        return err = "state format version " + std::to_string(h.version) + " (this library reads version 1)", false;
    if (h.checksum != header_checksum(h)) return err = "the header's checksum does not match its bytes", false;
    return true;
}

// a device buffer for a batch of blocks, freed with its scope
struct DeviceBuffer {
    uint8_t *p = nullptr;
    ~DeviceBuffer() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace
}  // namespace gv

using namespace gv;

extern "C" {

int gv_model_save_state(gv_model *g, const char *path, int append, const gv_state_info *info) {
    GV_REQUIRE(g && path && *path && info, "gv_model_save_state: bad arguments");
    Model &m = model_of(g);
    const auto &c = m.c;
    GV_REQUIRE(c.head_dim % 16 == 0, "gv_model_save_state: head_dim must be a multiple of 16");
    const Shapes s = shapes_of(m);
    StateHeader h{};
    std::memcpy(h.magic, kMagic, sizeof kMagic);
    h.version = kVersion;
    h.header_size = sizeof(StateHeader);
    h.fingerprint = fingerprint_of(m, *info);
    h.conv_id = info->conv_id;
    h.gen = 1;
    h.position = m.pos;
    h.extra = info->extra;
    h.rope_delta = info->rope_delta;
    h.n_images = 0;
    h.image_cap = 16;
    h.kv_elem = s.elem;
    h.n_attn = static_cast<uint32_t>(m.attn_layers.size());
    h.kv_heads = static_cast<uint32_t>(c.n_kv_heads);
    h.kv_row = s.kv_row;
    h.hidden = static_cast<uint32_t>(c.hidden);
    h.has_hidden = info->hidden && (info->has_mtp || m.has_mtp) && m.pos > 0 ? 1 : 0;
    h.block = kStateBlock;
    h.conv_n = conv_n_of(m);
    h.gdn_n = gdn_n_of(m);
    h.fixed_offset = kHeaderBytes;
    h.block_bytes = s.block_bytes;
    // an append: the file holds an earlier state of this conversation in this shape (state.cpp:283-299); the blocks
    // are written again from the one that holds the last saved position
    int first_block = 0;
    bool in_place = false;
    if (append) {
        StateIo f;
        StateHeader old{};
        std::string e;
        if (f.open(path, StateIo::kRead) && read_header(f, old, e) && old.fingerprint == h.fingerprint &&
            old.conv_id == h.conv_id && old.position <= h.position && h.n_images <= old.image_cap &&
            old.block == h.block && old.block_bytes == h.block_bytes && old.fixed_offset == h.fixed_offset) {
            h.image_cap = old.image_cap;
            h.gen = old.gen + 1;
            first_block = std::max(0, old.position - 1) / kStateBlock;
            in_place = true;
        }
    }
    const Layout L = layout_of(h);
    h.fixed_bytes = L.fixed_bytes;
    h.kv_offset = L.kv_offset;
    h.checksum = header_checksum(h);

    const std::string target = in_place ? std::string(path) : std::string(path) + ".tmp";
    StateIo f;
    if (!f.open(target, in_place ? StateIo::kUpdate : StateIo::kCreate)) {
        set_error("gv_model_save_state: cannot write " + target);
        return GV_STATE_E_IO;
    }
    auto fail = [&](int code, const char *what) {
        f.shut();
        if (!in_place) std::remove(target.c_str());
        set_error(std::string("gv_model_save_state: ") + what + " (" + target + ")");
        return code;
    };
    {   // the fixed part: gen first; gen last once the rest is on the disk
        std::vector<uint8_t> head(static_cast<size_t>(L.conv - h.fixed_offset), 0);
        std::memcpy(head.data(), &h.gen, sizeof h.gen);
        if (h.has_hidden) std::memcpy(head.data() + (L.hidden - h.fixed_offset), info->hidden, size_t{h.hidden} * 4);
        std::vector<float> conv, rec;
        if (gdn_states_io(m, conv, rec, true) != 0) return fail(GV_STATE_E_IO, "cannot read the layers' states");
        if (!f.put(h.fixed_offset, head.data(), head.size()) || !f.put(L.conv, conv.data(), conv.size() * 4) ||
            !f.put(L.gdn, rec.data(), rec.size() * 4) || !f.flush() || !f.put(L.trail, &h.gen, sizeof h.gen))
            return fail(GV_STATE_E_IO, "writing the fixed part (generation, hidden row, layer states) failed");
    }
    const int blocks = (m.pos + kStateBlock - 1) / kStateBlock;
    if (blocks > first_block) {
        const size_t bb = static_cast<size_t>(h.block_bytes);
        const int per = static_cast<int>(std::max<size_t>(1, kIoBatch / bb));
        const size_t buf_bytes = static_cast<size_t>(std::min(per, blocks - first_block)) * bb;
        DeviceBuffer dbuf;
        if (hipMalloc(&dbuf.p, buf_bytes) != hipSuccess) {
            dbuf.p = nullptr;
            return fail(GV_STATE_E_MEMORY, "no device memory for a batch of the KV cache's blocks");
        }
        std::vector<uint8_t> buf(buf_bytes);
        const hipStream_t st = stream();
        for (int b0 = first_block; b0 < blocks; b0 += per) {
            const int nb = std::min(per, blocks - b0);
            launch_blocks<true>(m, kStateBlock, b0, nb, m.pos, dbuf.p, st);
            if (hipGetLastError() != hipSuccess ||
                hipMemcpyAsync(buf.data(), dbuf.p, static_cast<size_t>(nb) * bb, hipMemcpyDeviceToHost, st) != hipSuccess ||
                hipStreamSynchronize(st) != hipSuccess)
                return fail(GV_STATE_E_IO, "cannot read the KV cache from the device");
            if (!f.put(h.kv_offset + static_cast<uint64_t>(b0) * h.block_bytes, buf.data(), static_cast<size_t>(nb) * bb))
                return fail(GV_STATE_E_IO, "writing the KV blocks failed");
        }
    }
    if (!f.flush() || !f.put(0, &h, sizeof h) || !f.flush())   // the header last, once what it names is written
        return fail(GV_STATE_E_IO, "writing the header failed");
    f.shut();
    if (!in_place && std::rename(target.c_str(), path) != 0) {
        std::remove(target.c_str());
        set_error(std::string("gv_model_save_state: cannot move ") + target + " to " + path);
        return GV_STATE_E_IO;
    }
    return 0;
}

int gv_model_load_state(gv_model *g, const char *path, gv_state_info *info) {
    GV_REQUIRE(g && path && *path && info, "gv_model_load_state: bad arguments");
    Model &m = model_of(g);
    const auto &c = m.c;
    GV_REQUIRE(c.head_dim % 16 == 0, "gv_model_load_state: head_dim must be a multiple of 16");
    // whatever the failure, the conversation is empty after it (state.cpp:376-380: Model::reset, the Gated DeltaNet
    // states zero)
    auto reset = [&] {
        m.pos = 0;
        m.last_n = 0;
        m.mtp_last_n = 0;   // no MTP pass of the loaded conversation exists yet
        info->has_hidden = 0;
        return gdn_zero(m);
    };
    if (reset() != 0) return GV_STATE_E_IO;
    auto refuse = [&](int code, const std::string &e) {
        (void)reset();
        set_error("gv_model_load_state: " + e);
        return code;
    };
    StateIo f;
    if (!f.open(path, StateIo::kRead)) return refuse(GV_STATE_E_IO, std::string("cannot open ") + path);
    StateHeader h{};
    std::string e;
    if (!read_header(f, h, e)) return refuse(GV_STATE_E_FORMAT, e);
    const Shapes s = shapes_of(m);
    if (h.fingerprint != fingerprint_of(m, *info) || h.kv_elem != s.elem ||
        h.n_attn != static_cast<uint32_t>(m.attn_layers.size()) || h.kv_heads != static_cast<uint32_t>(c.n_kv_heads) ||
        h.kv_row != s.kv_row || h.hidden != static_cast<uint32_t>(c.hidden) || h.conv_n != conv_n_of(m) ||
        h.gdn_n != gdn_n_of(m) || h.block == 0 || h.block > (1u << 24))
        return refuse(GV_STATE_E_FORMAT, "the file's model fingerprint, layer shapes or KV element type differ from "
                                         "this model's");
    if (h.position < 0 || h.position >= c.max_ctx)
        return refuse(GV_STATE_E_ARG, "the file holds " + std::to_string(h.position) + " positions; this model's "
                                          "context is " + std::to_string(c.max_ctx));
    const Layout L = layout_of(h);
    const uint64_t B = h.block;
    const int blocks = static_cast<int>((static_cast<uint64_t>(h.position) + B - 1) / B);
    if (L.fixed_bytes != h.fixed_bytes || L.kv_offset != h.kv_offset || h.n_images > h.image_cap ||
        h.block_bytes != 2 * static_cast<uint64_t>(m.attn_layers.size()) * B * (uint64_t{s.kv_row} * s.elem + s.scale_bytes) ||
        f.length() < h.kv_offset + static_cast<uint64_t>(blocks) * h.block_bytes)
        return refuse(GV_STATE_E_IO, "the file ends before the parts its header names");
    uint64_t lead = 0, trail = 0;
    if (!f.get(h.fixed_offset, &lead, 8) || !f.get(L.trail, &trail, 8) || lead != h.gen || trail != h.gen)
        return refuse(GV_STATE_E_IO, "the fixed part's generation marks disagree with the header (a save did not finish)");
    // images need a vision encoder's rotary positions, which this model does not compute
    if (h.n_images != 0)
        return refuse(GV_STATE_E_FORMAT, "the file holds image positions; this model has no vision encoder");
    if (h.has_hidden && info->hidden && !f.get(L.hidden, info->hidden, size_t{h.hidden} * 4))
        return refuse(GV_STATE_E_IO, "reading the hidden row failed");
    {
        std::vector<float> conv(static_cast<size_t>(h.conv_n)), rec(static_cast<size_t>(h.gdn_n));
        if (!f.get(L.conv, conv.data(), conv.size() * 4) || !f.get(L.gdn, rec.data(), rec.size() * 4))
            return refuse(GV_STATE_E_IO, "reading the layer states failed");
        if (gdn_states_io(m, conv, rec, false) != 0) return refuse(GV_STATE_E_IO, "cannot copy the layers' states");
    }
    if (blocks > 0) {
        const size_t bb = static_cast<size_t>(h.block_bytes);
        const int per = static_cast<int>(std::max<size_t>(1, kIoBatch / bb));
        const size_t buf_bytes = static_cast<size_t>(std::min(per, blocks)) * bb;
        DeviceBuffer dbuf;
        if (hipMalloc(&dbuf.p, buf_bytes) != hipSuccess) {
            dbuf.p = nullptr;
            return refuse(GV_STATE_E_MEMORY, "no device memory for a batch of the KV cache's blocks");
        }
        std::vector<uint8_t> buf(buf_bytes);
        const hipStream_t st = stream();
        for (int b0 = 0; b0 < blocks; b0 += per) {
            const int nb = std::min(per, blocks - b0);
            if (!f.get(h.kv_offset + static_cast<uint64_t>(b0) * h.block_bytes, buf.data(), static_cast<size_t>(nb) * bb))
                return refuse(GV_STATE_E_IO, "reading the KV blocks failed");
            if (hipMemcpyAsync(dbuf.p, buf.data(), static_cast<size_t>(nb) * bb, hipMemcpyHostToDevice, st) != hipSuccess)
                return refuse(GV_STATE_E_IO, "cannot copy the KV cache to the device");
            launch_blocks<false>(m, static_cast<int>(B), b0, nb, h.position, dbuf.p, st);
            if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
                return refuse(GV_STATE_E_IO, "cannot copy the KV cache to the device");
        }
    }
    m.pos = h.position;
    m.last_n = 0;
    info->has_hidden = h.has_hidden && info->hidden ? 1 : 0;
    info->conv_id = h.conv_id;
    info->extra = h.extra;
    info->rope_delta = h.rope_delta;
    return 0;
}

}  // extern "C"
