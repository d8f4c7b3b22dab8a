// pack.hip - a geode-pack opened on the host (the reference's Pack::open, engine/src/pack.cpp:39-308) and its tensors
// adopted by the GPU model.
//
// A pack is a directory: geode.json (the manifest: format "geode-pack" v1, the architecture, the files with their
// sizes, the model's config, the tensor table {name: type, shape, file, offset, global} and the expert table: per
// layer a file and either offset + stride + format or per-expert offsets and formats) and the files it lists
// (dense.bin, the experts' files). Opening checks what the reference checks: the files present at their sizes, the
// geometry, every tensor's type, shape and extent inside its file, the expert table and the experts' scales. An
// expert block is its gate_up rows then its down rows (pack.cpp:329-333); a pack whose q4 experts are in the tiled
// "tile8" layout (formats.q4.layout, kernels.hpp:49-56) has them turned back into rows here (the inverse of
// to_tile8, kernels.cpp:971-991) before the device makes its own layout of them.
//
// Host code only: the JSON reader, the table and the file reads; the bytes go to the device through
// gv_model_adopt.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/geode_verify.h"
#include "common.hpp"
#include "model.hpp"

namespace gv {
namespace {

// ---------------------------------------------------------------- JSON (the manifest's subset: all of RFC 8259)
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string s;
    std::vector<Json> a;
    std::map<std::string, Json> o;

    const Json &operator[](const std::string &key) const {
        static const Json none;
        if (kind != Obj) return none;
        const auto it = o.find(key);
        return it == o.end() ? none : it->second;
    }
    const Json &at(size_t i) const {
        static const Json none;
        return kind == Arr && i < a.size() ? a[i] : none;
    }
    size_t size() const { return kind == Arr ? a.size() : kind == Obj ? o.size() : 0; }
    std::string str(const std::string &fallback = "") const { return kind == Str ? s : fallback; }
    int64_t i64(int64_t fallback = 0) const { return kind == Num ? static_cast<int64_t>(num) : fallback; }
    double f64(double fallback = 0.0) const { return kind == Num ? num : fallback; }
};

class JsonReader {
public:
    JsonReader(const char *p, size_t n) : p_(p), begin_(p), end_(p + n) {}
    bool read(Json &out, std::string &err) {
        if (!value(out, 0) || (skip(), p_ != end_)) {
            if (err_.empty()) err_ = "trailing characters";
            err = err_ + " at byte " + std::to_string(p_ - begin_);
            return false;
        }
        return true;
    }

private:
    const char *p_, *begin_, *end_;
    std::string err_;

    bool fail(const char *what) {
        if (err_.empty()) err_ = what;
        return false;
    }
    void skip() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool literal(const char *w) {
        const size_t n = std::strlen(w);
        if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return fail("unexpected characters");
        p_ += n;
        return true;
    }
    static void utf8(uint32_t cp, std::string &out) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t &v) {
        if (end_ - p_ < 4) return fail("a short \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
            else return fail("a bad \\u escape");
        }
        return true;
    }
    bool string(std::string &out) {
        ++p_;   // the opening quote
        while (p_ < end_ && *p_ != '"') {
            const unsigned char c = static_cast<unsigned char>(*p_);
            if (c < 0x20) return fail("a control character in a string");
            if (c != '\\') {
                out += *p_++;
                continue;
            }
            if (++p_ == end_) break;
            const char e = *p_++;
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                    const char *save = p_;
                    p_ += 2;
                    uint32_t lo;
                    if (!hex4(lo)) return false;
                    if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    else p_ = save;
                }
                utf8(cp, out);
                break;
            }
            default: return fail("a bad escape");
            }
        }
        if (p_ == end_) return fail("an unterminated string");
        ++p_;
        return true;
    }
    bool number(double &out) {
        const char *s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ == end_ || !((*p_ >= '0' && *p_ <= '9'))) return fail("a bad number");
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                             *p_ == '-'))
            ++p_;
        const std::string text(s, p_);
        char *stop = nullptr;
        out = std::strtod(text.c_str(), &stop);
        if (!stop || *stop != '\0') return fail("a bad number");
        return true;
    }
    bool value(Json &v, int depth) {
        if (depth > 64) return fail("nested too deeply");
        skip();
        if (p_ == end_) return fail("unexpected end");
        switch (*p_) {
        case '{': {
            ++p_;
            v.kind = Json::Obj;
            skip();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            while (true) {
                skip();
                if (p_ == end_ || *p_ != '"') return fail("a key expected");
                std::string key;
                if (!string(key)) return false;
                skip();
                if (p_ == end_ || *p_ != ':') return fail("':' expected");
                ++p_;
                Json item;
                if (!value(item, depth + 1)) return false;
                v.o[key] = std::move(item);
                skip();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return fail("',' or '}' expected");
            }
        }
        case '[': {
            ++p_;
            v.kind = Json::Arr;
            skip();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            while (true) {
                Json item;
                if (!value(item, depth + 1)) return false;
                v.a.push_back(std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return fail("',' or ']' expected");
            }
        }
        case '"': v.kind = Json::Str; return string(v.s);
        case 't': v.kind = Json::Bool, v.b = true; return literal("true");
        case 'f': v.kind = Json::Bool, v.b = false; return literal("false");
        case 'n': v.kind = Json::Null; return literal("null");
        default: v.kind = Json::Num; return number(v.num);
        }
    }
};

// ---------------------------------------------------------------- the table (kernels.cpp:858-902)
enum Type { T_F32 = 0, T_BF16 = 1, T_Q2 = 2, T_Q3 = 3, T_NVFP4 = 4, T_Q8 = 5, T_Q4 = 6, T_UNKNOWN = 7, T_Q4I = 8 };

int type_of(const std::string &n) {
    static const char *names[] = {"f32", "bf16", "q2", "q3", "nvfp4", "q8", "q4", "", "q4i"};
    for (int i = 0; i < 9; ++i)
        if (i != T_UNKNOWN && n == names[i]) return i;
    return T_UNKNOWN;
}
bool quantized(int t) { return t == T_Q2 || t == T_Q3 || t == T_NVFP4 || t == T_Q8 || t == T_Q4 || t == T_Q4I; }
int block_code_bytes(int t) {
    switch (t) {
    case T_Q2: return 4;
    case T_Q3: return 6;
    case T_NVFP4: return 8;
    case T_Q4: return 8;
    case T_Q4I: return 8;
    case T_Q8: return 16;
    default: return 0;
    }
}
uint64_t row_bytes(int t, int64_t cols) { return static_cast<uint64_t>(cols / 16) * static_cast<uint64_t>(block_code_bytes(t) + 1); }

struct Tensor {
    int type = T_UNKNOWN;
    std::vector<int64_t> shape;
    int64_t rows = 0, cols = 0;
    int file = -1;
    uint64_t offset = 0;
    float global = 1.0f;
    uint64_t bytes() const {
        return quantized(type) ? static_cast<uint64_t>(rows) * row_bytes(type, cols)
                               : static_cast<uint64_t>(rows * cols) * (type == T_F32 ? 4 : 2);
    }
};

struct ExpertLayer {
    int file = -1;
    uint64_t offset = 0, stride = 0;   // uniform: expert e at offset + e x stride
    int type = T_UNKNOWN;
    std::vector<uint64_t> offsets;     // mixed formats: per expert
    std::vector<int> types;
};

// a file read at offsets
struct ReadFile {
    int fd = -1;
    ~ReadFile() {
        if (fd >= 0) ::close(fd);
    }
    bool open(const std::string &path) {
        fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        return fd >= 0;
    }
    bool read(uint64_t off, void *data, size_t n) const {
        auto *p = static_cast<uint8_t *>(data);
        while (n > 0) {
            const ssize_t r = ::pread(fd, p, std::min<size_t>(n, size_t{1} << 30), static_cast<off_t>(off));
            if (r <= 0) return false;
            p += r, off += static_cast<uint64_t>(r), n -= static_cast<size_t>(r);
        }
        return true;
    }
};

bool file_size(const std::string &path, uint64_t &size) {
    struct stat s {};
    if (::stat(path.c_str(), &s) != 0) return false;
    size = static_cast<uint64_t>(s.st_size);
    return true;
}

// FNV-1a from the reference's start (state.cpp:68-73, 1469598103934665603: its pack print starts there)
uint64_t fnv(const void *data, size_t n, uint64_t h = 1469598103934665603ull) {
    const auto *p = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

}  // namespace
}  // namespace gv

using namespace gv;

struct gv_pack {
    std::string dir;
    Json m;
    uint64_t print = 1;
    std::string arch;
    // the geometry (pack.cpp:90-160)
    int hidden = 0, n_layers = 0, vocab = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, rope_dim = 0;
    int gdn_k_heads = 0, gdn_v_heads = 0, gdn_k_dim = 0, gdn_v_dim = 0, conv_kernel = 0;
    int n_experts = 0, top_k = 0, moe_ff = 0, shared_ff = 0;
    float eps = 1e-6f, rope_theta = 10000.0f;
    bool dense = false, tile8 = false, mtp = false;
    std::vector<bool> attention;
    std::vector<std::string> files;   // the files present
    std::vector<uint64_t> sizes;
    std::map<std::string, Tensor> tensors;
    std::vector<ExpertLayer> experts;   // [n_layers] (+ the MTP layer's)

    const Tensor *find(const std::string &name) const {
        const auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
    int file_index(const std::string &name) const {
        for (size_t i = 0; i < files.size(); ++i)
            if (files[i] == name) return static_cast<int>(i);
        return -1;
    }
};

namespace gv {
namespace {

int geti(const Json &v, const char *key, int fallback = 0) { return static_cast<int>(v[key].i64(fallback)); }

// Pack::open (pack.cpp:39-308) without reading dense.bin into memory: the tensors are read from their files when
// adopted
bool open_pack(gv_pack &P, const std::string &dir, std::string &err) {
    P.dir = dir;
    const std::string mpath = dir + "/geode.json";
    std::string text;
    {
        std::FILE *f = std::fopen(mpath.c_str(), "rb");
        if (!f) return err = "no geode.json in " + dir, false;
        char buf[1 << 16];
        size_t n;
        while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
        std::fclose(f);
    }
    const uint64_t h = fnv(text.data(), text.size());   // Model::fingerprint's pack print (state.cpp:227-238)
    P.print = h ? h : 1;
    std::string perr;
    if (!JsonReader(text.data(), text.size()).read(P.m, perr)) return err = "geode.json: " + perr, false;
    const Json &m = P.m;
    if (m["format"].str() != "geode-pack" || m["version"].i64() != 1)
        return err = "not a geode-pack v1 (format '" + m["format"].str() + "')", false;
    P.arch = m["arch"].str();
    const bool gemma = P.arch == "gemma4";
    if (P.arch != "qwen35moe" && P.arch != "qwen35" && !gemma) return err = "unknown architecture '" + P.arch + "'", false;

    // the files: present at their sizes; an optional one may be missing, its tensors then absent
    const Json &files = m["files"];
    std::vector<std::string> missing;
    for (size_t i = 0; i < files.size(); ++i) {
        const Json &f = files.at(i);
        const std::string name = f["name"].str();
        uint64_t size = 0;
        const bool there = file_size(dir + "/" + name, size);
        if (f["optional"].kind == Json::Bool && f["optional"].b && !there) {
            missing.push_back(name);
            continue;
        }
        if (!there) return err = "cannot open " + dir + "/" + name, false;
        if (static_cast<int64_t>(size) != f["size"].i64())
            return err = name + ": " + std::to_string(size) + " bytes, expected " + std::to_string(f["size"].i64()), false;
        P.files.push_back(name);
        P.sizes.push_back(size);
    }

    // the geometry
    const Json &c = m["config"];
    P.hidden = geti(c, "hidden_size");
    P.n_layers = geti(c, "num_hidden_layers");
    P.vocab = geti(c, "vocab_size");
    P.eps = static_cast<float>(c["rms_norm_eps"].f64(1e-6));
    P.n_heads = geti(c, "num_attention_heads");
    P.n_kv_heads = geti(c, "num_key_value_heads");
    P.head_dim = geti(c, "head_dim");
    const Json &rope = c["rope_parameters"];
    P.rope_theta = static_cast<float>(rope["rope_theta"].f64(10000.0));
    P.rope_dim = static_cast<int>(P.head_dim * rope["partial_rotary_factor"].f64(1.0));
    P.gdn_k_heads = geti(c, "linear_num_key_heads");
    P.gdn_v_heads = geti(c, "linear_num_value_heads");
    P.gdn_k_dim = geti(c, "linear_key_head_dim");
    P.gdn_v_dim = geti(c, "linear_value_head_dim");
    P.conv_kernel = geti(c, "linear_conv_kernel_dim");
    P.dense = P.arch == "qwen35" || gemma;
    P.n_experts = gemma ? 0 : geti(c, "num_experts");
    P.top_k = gemma ? 0 : geti(c, "num_experts_per_tok");
    P.moe_ff = gemma ? 0 : geti(c, "moe_intermediate_size");
    P.shared_ff = geti(c, P.arch == "qwen35" ? "intermediate_size" : "shared_expert_intermediate_size");
    const Json &types = c["layer_types"];
    if (P.n_layers <= 0 || P.n_layers > 1024 || static_cast<int>(types.size()) != P.n_layers)
        return err = "geode.json: layer_types does not match num_hidden_layers", false;
    for (int l = 0; l < P.n_layers; ++l) P.attention.push_back(types.at(static_cast<size_t>(l)).str() == "full_attention");
    const bool moe_ok = P.dense ? P.n_experts == 0 && (gemma || (P.shared_ff > 0 && P.shared_ff % 16 == 0))
                                : P.top_k > 0 && P.top_k <= P.n_experts;
    if (P.hidden <= 0 || P.hidden % 16 || !moe_ok || P.gdn_v_heads % std::max(1, P.gdn_k_heads) ||
        P.n_heads % std::max(1, P.n_kv_heads) || P.rope_dim % 2)
        return err = "geode.json: inconsistent model geometry", false;

    // the tensor table: every shape and extent checked before anything is read
    const Json &tensors = m["tensors"];
    if (tensors.kind != Json::Obj) return err = "geode.json: no tensor table", false;
    bool any_dense = false;
    for (const auto &[name, t] : tensors.o) {
        if (std::find(missing.begin(), missing.end(), t["file"].str()) != missing.end()) continue;
        Tensor x;
        x.type = type_of(t["type"].str());
        if (x.type == T_UNKNOWN) return err = name + ": unknown type '" + t["type"].str() + "'", false;
        bool shape_ok = true;
        for (size_t i = 0; i < t["shape"].size(); ++i) {
            const int64_t d = t["shape"].at(i).i64();
            shape_ok &= d > 0 && d < (int64_t{1} << 31);
            x.shape.push_back(d);
        }
        if (x.shape.empty()) x.shape.push_back(1);
        x.rows = x.shape[0];
        x.cols = 1;
        for (size_t i = 1; i < x.shape.size() && shape_ok; ++i) {
            x.cols *= x.shape[i];
            shape_ok &= x.cols < (int64_t{1} << 40);
        }
        if (x.shape.size() == 1) {
            x.cols = x.rows;
            x.rows = 1;
        }
        const int64_t off = t["offset"].i64();
        if (!shape_ok || off < 0 || static_cast<double>(x.rows) * static_cast<double>(x.cols) > 1099511627776.0)
            return err = name + ": a shape or an offset out of range", false;
        x.file = P.file_index(t["file"].str());
        if (x.file < 0) return err = "geode.json names a file it does not list: " + t["file"].str(), false;
        x.offset = static_cast<uint64_t>(off);
        x.global = static_cast<float>(t["global"].f64(1.0));
        if (quantized(x.type) && x.cols % 16) return err = name + ": columns not a multiple of 16", false;
        const uint64_t fsize = P.sizes[static_cast<size_t>(x.file)];
        if (x.offset > fsize || x.bytes() > fsize - x.offset) return err = name + ": runs past the end of " + t["file"].str(), false;
        any_dense |= t["file"].str() == "dense.bin";
        P.tensors.emplace(name, std::move(x));
    }
    if (!any_dense) return err = "geode.json: no tensors in dense.bin", false;
    const Tensor *embed = P.find("embed_tokens.weight");
    if (!embed || !quantized(embed->type) || embed->cols != P.hidden) return err = "geode.json: no usable embed_tokens.weight", false;

    // the experts
    const Json &el = m["experts"]["layers"];
    if (static_cast<int>(el.size()) != (P.dense ? 0 : P.n_layers))
        return err = "geode.json: the expert table does not cover every layer", false;
    auto expert_layer = [&](const Json &e, int l) -> bool {
        ExpertLayer x;
        x.file = P.file_index(e["file"].str());
        if (x.file < 0) return err = "geode.json names a file it does not list: " + e["file"].str(), false;
        x.offset = static_cast<uint64_t>(e["offset"].i64());
        if (e["stride"].kind == Json::Num) {
            x.stride = static_cast<uint64_t>(e["stride"].i64());
            x.type = type_of(e["format"].str());
        } else {
            for (size_t i = 0; i < e["offsets"].size(); ++i) {
                x.offsets.push_back(static_cast<uint64_t>(e["offsets"].at(i).i64()));
                x.types.push_back(type_of(e["formats"].at(i).str()));
            }
            if (static_cast<int>(x.offsets.size()) != P.n_experts)
                return err = "geode.json: layer " + std::to_string(l) + " lists the wrong number of experts", false;
        }
        P.experts.push_back(std::move(x));
        const std::string scales = l < P.n_layers ? "layers." + std::to_string(l) + ".mlp.experts.scales"
                                                  : "mtp.layers.0.mlp.experts.scales";
        const Tensor *s = P.find(scales);
        if (!s || s->type != T_F32 || s->rows != P.n_experts || s->cols != 2)
            return err = "geode.json: no expert scales for layer " + std::to_string(l), false;
        return true;
    };
    for (int l = 0; l < (P.dense ? 0 : P.n_layers); ++l)
        if (!expert_layer(el.at(static_cast<size_t>(l)), l)) return false;
    bool any_q3 = false;
    for (const auto &[name, t] : P.tensors) any_q3 |= t.type == T_Q3;
    for (const auto &x : P.experts) {
        any_q3 |= x.type == T_Q3;
        for (int t : x.types) any_q3 |= t == T_Q3;
    }
    if (any_q3 && m["formats"]["q3"]["high_bits"].str() != "value order")
        return err = "geode.json: q3 with the old bit planes", false;
    P.tile8 = m["formats"]["q4"]["layout"].str() == "tile8";
    if (m["mtp"].kind == Json::Obj) {
        if (!P.dense && !expert_layer(m["mtp"]["experts"], P.n_layers)) return false;
        P.mtp = true;
    }
    return true;
}

// tile8 (kernels.cpp:971-991) back to the pack's rows: per 32-row tile, code word j of chunk c of quad i (four rows'
// 32-bit words, affine codes) at ((c * 8 + j) * 8 + i) * 16 + 4 r, then the scales, block b of chunk c of row r of
// quad i at 1024 * nch + (c * 8 + i) * 16 + 4 b + r; an affine nibble c' is the pack's code c' - 8 (c' >= 8) or
// 15 - c'.
void untile8(int64_t rows, int64_t cols, const uint8_t *src, uint8_t *dst) {
    const size_t rb = static_cast<size_t>(row_bytes(T_Q4, cols)), nch = static_cast<size_t>(cols / 64);
    const size_t code = static_cast<size_t>(cols / 2);
    uint8_t from[256];
    for (int b = 0; b < 256; ++b) {
        int v = 0;
        for (int k = 0; k < 2; ++k) {
            const int c = (b >> (4 * k)) & 15;
            v |= (c >= 8 ? c - 8 : 15 - c) << (4 * k);
        }
        from[b] = static_cast<uint8_t>(v);
    }
    for (int64_t t0 = 0; t0 < rows; t0 += 32) {
        const uint8_t *g = src + static_cast<size_t>(t0) * rb;
        uint8_t *out = dst + static_cast<size_t>(t0) * rb;
        for (size_t i = 0; i < 8; ++i)
            for (size_t r = 0; r < 4; ++r) {
                uint8_t *row = out + (4 * i + r) * rb;
                for (size_t c = 0; c < nch; ++c) {
                    for (size_t j = 0; j < 8; ++j)
                        for (size_t k = 0; k < 4; ++k) row[(c * 8 + j) * 4 + k] = from[g[((c * 8 + j) * 8 + i) * 16 + r * 4 + k]];
                    for (size_t b = 0; b < 4; ++b) row[code + c * 4 + b] = g[1024 * nch + (c * 8 + i) * 16 + b * 4 + r];
                }
            }
    }
}

struct Reader {   // the pack's files, opened once for a load
    const gv_pack &P;
    std::vector<std::unique_ptr<ReadFile>> f;
    explicit Reader(const gv_pack &p) : P(p) {}
    bool open(std::string &err) {
        for (const auto &name : P.files) {
            auto rf = std::make_unique<ReadFile>();
            if (!rf->open(P.dir + "/" + name)) return err = "cannot open " + P.dir + "/" + name, false;
            f.push_back(std::move(rf));
        }
        return true;
    }
    bool tensor(const Tensor &t, std::vector<uint8_t> &out) const {
        out.resize(t.bytes());
        return f[static_cast<size_t>(t.file)]->read(t.offset, out.data(), out.size());
    }
};

}  // namespace
}  // namespace gv

extern "C" {

gv_pack *gv_pack_open(const char *dir, char *err, int err_len) {
    auto put = [&](const std::string &e) {
        if (err && err_len > 0) {
            std::strncpy(err, e.c_str(), static_cast<size_t>(err_len) - 1);
            err[err_len - 1] = '\0';
        }
        set_error("gv_pack_open: " + e);
    };
    if (!dir) {
        put("null directory");
        return nullptr;
    }
    auto P = std::make_unique<gv_pack>();
    std::string e;
    if (!open_pack(*P, dir, e)) {
        put(e);
        return nullptr;
    }
    return P.release();
}

void gv_pack_close(gv_pack *p) { delete p; }

uint64_t gv_pack_print(const gv_pack *p) { return p ? p->print : 0; }

int gv_pack_model_config(const gv_pack *p, int max_ctx, int max_rows, int kv_int8, gv_model_config *out) {
    GV_REQUIRE(p && out, "gv_pack_model_config: null pointer");
    GV_REQUIRE(p->arch == "qwen35moe", "gv_pack_model_config: the GPU model takes qwen35moe packs (this one is '" +
                                           p->arch + "')");
    bool any_gdn = false;
    for (int l = 0; l < p->n_layers; ++l) any_gdn = any_gdn || !p->attention[static_cast<size_t>(l)];
    GV_REQUIRE(!any_gdn || p->n_layers <= 256, "gv_pack_model_config: a Gated DeltaNet model of more than 256 layers");
    GV_REQUIRE(p->shared_ff == p->moe_ff, "gv_pack_model_config: the shared expert's width differs from the experts'");
    gv_model_config c{};
    c.hidden = p->hidden;
    c.vocab = p->vocab;
    c.n_layers = p->n_layers;
    c.n_experts = p->n_experts;
    c.top_k = p->top_k;
    c.moe_ff = p->moe_ff;
    c.shared_ff = p->shared_ff;
    c.n_heads = p->n_heads;
    c.n_kv_heads = p->n_kv_heads;
    c.head_dim = p->head_dim;
    c.rope_dim = p->rope_dim;
    c.rope_theta = p->rope_theta;
    c.eps = p->eps;
    c.max_ctx = max_ctx;
    c.max_rows = max_rows;
    c.kv_int8 = kv_int8;
    c.mtp = p->mtp ? 1 : 0;   // ModelConfig::mtp_layers (pack.cpp:303-305); a caller may set it to 0 (no drafting)
    if (any_gdn) {   // ModelConfig's Gated DeltaNet shape (pack.cpp:96-100), the layers not "full_attention"
        c.gdn_k_heads = p->gdn_k_heads;
        c.gdn_v_heads = p->gdn_v_heads;
        c.gdn_k_dim = p->gdn_k_dim;
        c.gdn_v_dim = p->gdn_v_dim;
        c.conv_kernel = p->conv_kernel;
        for (int l = 0; l < p->n_layers; ++l) c.gdn_layers[l] = p->attention[static_cast<size_t>(l)] ? 0 : 1;
    }
    *out = c;
    return 0;
}

int gv_pack_tensor(const gv_pack *p, const char *name, gv_pack_tensor_info *out) {
    GV_REQUIRE(p && name && out, "gv_pack_tensor: null pointer");
    const Tensor *t = p->find(name);
    GV_REQUIRE(t, std::string("gv_pack_tensor: the pack has no ") + name);
    out->type = t->type;
    out->rows = t->rows;
    out->cols = t->cols;
    out->file = t->file;
    out->offset = t->offset;
    out->bytes = t->bytes();
    out->global = t->global;
    return 0;
}

int gv_pack_expert(const gv_pack *p, int layer, int expert, int *file, uint64_t *offset, int *type) {
    GV_REQUIRE(p && file && offset && type, "gv_pack_expert: null pointer");
    GV_REQUIRE(layer >= 0 && layer < static_cast<int>(p->experts.size()) && expert >= 0 && expert < p->n_experts,
               "gv_pack_expert: no such expert");
    const ExpertLayer &x = p->experts[static_cast<size_t>(layer)];
    *file = x.file;
    if (x.stride) {
        *offset = x.offset + static_cast<uint64_t>(expert) * x.stride;
        *type = x.type;
    } else {
        *offset = x.offsets[static_cast<size_t>(expert)];
        *type = x.types[static_cast<size_t>(expert)];
    }
    return 0;
}

int gv_pack_tile8(const gv_pack *p) { return p && p->tile8 ? 1 : 0; }

int gv_q4_untile8(int64_t rows, int64_t cols, const uint8_t *src, uint8_t *dst) {
    GV_REQUIRE(src && dst && src != dst, "gv_q4_untile8: bad pointers");
    GV_REQUIRE(rows > 0 && rows % 32 == 0 && cols > 0 && cols % 64 == 0, "gv_q4_untile8: rows % 32 and cols % 64");
    untile8(rows, cols, src, dst);
    return 0;
}

int gv_model_load_pack(gv_model *g, const gv_pack *p) {
    GV_REQUIRE(g && p, "gv_model_load_pack: null pointer");
    gv_model_config want{};
    if (gv_pack_model_config(p, 0, 0, 0, &want) != 0) return -1;
    Reader rd(*p);
    std::string e;
    GV_REQUIRE(rd.open(e), "gv_model_load_pack: " + e);
    std::vector<uint8_t> buf, cat;
    // a tensor: its type and shape as the model takes it, then its bytes
    auto get = [&](const std::string &name, int type, int64_t rows, int64_t cols, const Tensor *&t) -> int {
        t = p->find(name);
        GV_REQUIRE(t, "gv_model_load_pack: the pack has no " + name);
        GV_REQUIRE(t->type == type && t->rows == rows && t->cols == cols,
                   "gv_model_load_pack: " + name + ": expected " + (type == T_Q4 ? "q4" : type == T_F32 ? "f32" : "bf16") +
                       " [" + std::to_string(rows) + ", " + std::to_string(cols) + "]");
        GV_REQUIRE(rd.tensor(*t, buf), "gv_model_load_pack: cannot read " + name);
        return 0;
    };
    // an f32 tensor of count values, whatever its shape (Model::bind_layer's f32, model.cpp:96-104)
    auto get_f32 = [&](const std::string &name, int64_t count, const Tensor *&t) -> int {
        t = p->find(name);
        GV_REQUIRE(t, "gv_model_load_pack: the pack has no " + name);
        GV_REQUIRE(t->type == T_F32 && t->rows * t->cols == count,
                   "gv_model_load_pack: " + name + ": expected f32 x " + std::to_string(count));
        GV_REQUIRE(rd.tensor(*t, buf), "gv_model_load_pack: cannot read " + name);
        return 0;
    };
    auto adopt = [&](int kind, int layer, int expert, const void *data, size_t bytes, const float *globals) -> int {
        return gv_model_adopt(g, kind, layer, expert, data, static_cast<int64_t>(bytes), globals);
    };
    const int64_t H = p->hidden, V = p->vocab, nh = p->n_heads, nkv = p->n_kv_heads, hd = p->head_dim, F = p->moe_ff;
    const Tensor *t = nullptr;
    for (const auto &[name, kind] : {std::make_pair(std::string("embed_tokens.weight"), GV_EMBED),
                                     std::make_pair(std::string("lm_head.weight"), GV_LM_HEAD)}) {
        if (get(name, T_Q4, V, H, t) != 0 || adopt(kind, 0, 0, buf.data(), buf.size(), &t->global) != 0) return -1;
    }
    if (get_f32("norm.weight", H, t) != 0 || adopt(GV_FINAL_NORM, 0, 0, buf.data(), buf.size(), nullptr) != 0)
        return -1;
    const int64_t nk = p->gdn_k_heads, nv = p->gdn_v_heads, dk = p->gdn_k_dim, dv = p->gdn_v_dim, K = p->conv_kernel;
    const int64_t conv_dim = 2 * nk * dk + nv * dv, vd = nv * dv;
    // a decoder layer's tensors under `pre` (the MTP layer's: "mtp.layers.0.", layer index n_layers, attention)
    auto load_layer = [&](int l, const std::string &pre, bool attention) -> int {
        struct F32 {
            const char *name;
            int kind;
            int64_t n;
        };
        for (const F32 &f : {F32{"input_layernorm.weight", GV_IN_NORM, H}, F32{"post_attention_layernorm.weight", GV_POST_NORM, H}})
            if (get_f32(pre + f.name, f.n, t) != 0 || adopt(f.kind, l, 0, buf.data(), buf.size(), nullptr) != 0)
                return -1;
        float gl[3];
        if (!attention) {   // a Gated DeltaNet layer (model.cpp:136-146)
            struct Q {
                const char *name;
                int kind;
                int64_t rows, cols;
            };
            for (const Q &q : {Q{"linear_attn.in_proj_qkv.weight", GV_GDN_QKV, conv_dim, H},
                               Q{"linear_attn.in_proj_z.weight", GV_GDN_Z, vd, H},
                               Q{"linear_attn.out_proj.weight", GV_GDN_OUT, H, vd}})
                if (get(pre + q.name, T_Q4, q.rows, q.cols, t) != 0 ||
                    adopt(q.kind, l, 0, buf.data(), buf.size(), &t->global) != 0)
                    return -1;
            for (const auto &[name, kind] : {std::make_pair("linear_attn.in_proj_a.weight", GV_GDN_A),
                                             std::make_pair("linear_attn.in_proj_b.weight", GV_GDN_B)})
                if (get(pre + name, T_BF16, nv, H, t) != 0 || adopt(kind, l, 0, buf.data(), buf.size(), nullptr) != 0)
                    return -1;
            for (const F32 &f : {F32{"linear_attn.A_log", GV_GDN_ALOG, nv}, F32{"linear_attn.dt_bias", GV_GDN_DTB, nv},
                                 F32{"linear_attn.conv1d.weight", GV_GDN_CONV, conv_dim * K},
                                 F32{"linear_attn.norm.weight", GV_GDN_NORM, dv}})
                if (get_f32(pre + f.name, f.n, t) != 0 || adopt(f.kind, l, 0, buf.data(), buf.size(), nullptr) != 0)
                    return -1;
        } else {
            for (const F32 &f : {F32{"self_attn.q_norm.weight", GV_Q_NORM, hd}, F32{"self_attn.k_norm.weight", GV_K_NORM, hd}})
                if (get_f32(pre + f.name, f.n, t) != 0 || adopt(f.kind, l, 0, buf.data(), buf.size(), nullptr) != 0)
                    return -1;
            // q | k | v rows in one matrix, a global each
            cat.clear();
            const int64_t qkv_rows[3] = {nh * hd * 2, nkv * hd, nkv * hd};
            const char *qkv_names[3] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight"};
            for (int i = 0; i < 3; ++i) {
                if (get(pre + qkv_names[i], T_Q4, qkv_rows[i], H, t) != 0) return -1;
                gl[i] = t->global;
                cat.insert(cat.end(), buf.begin(), buf.end());
            }
            if (adopt(GV_QKV, l, 0, cat.data(), cat.size(), gl) != 0) return -1;
            if (get(pre + "self_attn.o_proj.weight", T_Q4, H, nh * hd, t) != 0 ||
                adopt(GV_O, l, 0, buf.data(), buf.size(), &t->global) != 0)
                return -1;
        }
        if (get(pre + "mlp.gate.weight", T_BF16, p->n_experts, H, t) != 0 ||
            adopt(GV_ROUTER, l, 0, buf.data(), buf.size(), nullptr) != 0)
            return -1;
        if (get(pre + "mlp.shared_expert_gate.weight", T_BF16, 1, H, t) != 0 ||
            adopt(GV_SHARED_GATE, l, 0, buf.data(), buf.size(), nullptr) != 0)
            return -1;
        cat.clear();
        const int64_t sh_rows[3] = {F, F, H}, sh_cols[3] = {H, H, F};
        const char *sh_names[3] = {"mlp.shared_expert.gate_proj.weight", "mlp.shared_expert.up_proj.weight",
                                   "mlp.shared_expert.down_proj.weight"};
        for (int i = 0; i < 3; ++i) {
            if (get(pre + sh_names[i], T_Q4, sh_rows[i], sh_cols[i], t) != 0) return -1;
            gl[i] = t->global;
            cat.insert(cat.end(), buf.begin(), buf.end());
        }
        if (adopt(GV_SHARED_EXPERT, l, 0, cat.data(), cat.size(), gl) != 0) return -1;
        // the routed experts: the block (gate_up rows, down rows), its two globals from the layer's scales
        if (get(pre + "mlp.experts.scales", T_F32, p->n_experts, 2, t) != 0) return -1;
        const std::vector<float> scales(reinterpret_cast<const float *>(buf.data()),
                                        reinterpret_cast<const float *>(buf.data()) + 2 * p->n_experts);
        const uint64_t gu = static_cast<uint64_t>(2 * F) * row_bytes(T_Q4, H), dn = static_cast<uint64_t>(H) * row_bytes(T_Q4, F);
        std::vector<uint8_t> blk(gu + dn), rows(gu + dn);
        for (int ex = 0; ex < p->n_experts; ++ex) {
            int file, type;
            uint64_t off;
            if (gv_pack_expert(p, l, ex, &file, &off, &type) != 0) return -1;
            GV_REQUIRE(type == T_Q4, "gv_model_load_pack: layer " + std::to_string(l) + " expert " + std::to_string(ex) +
                                         ": the GPU model takes q4 experts");
            GV_REQUIRE(off <= p->sizes[static_cast<size_t>(file)] && gu + dn <= p->sizes[static_cast<size_t>(file)] - off,
                       "gv_model_load_pack: an expert runs past the end of " + p->files[static_cast<size_t>(file)]);
            GV_REQUIRE(rd.f[static_cast<size_t>(file)]->read(off, blk.data(), blk.size()),
                       "gv_model_load_pack: cannot read layer " + std::to_string(l) + " expert " + std::to_string(ex));
            const uint8_t *src = blk.data();
            if (p->tile8) {   // gate_up and down each tiled: back to rows
                GV_REQUIRE(H % 64 == 0 && F % 64 == 0 && H % 32 == 0 && (2 * F) % 32 == 0,
                           "gv_model_load_pack: tile8 experts need hidden and moe_ff multiples of 64");
                untile8(2 * F, H, blk.data(), rows.data());
                untile8(H, F, blk.data() + gu, rows.data() + gu);
                src = rows.data();
            }
            if (adopt(GV_EXPERT, l, ex, src, blk.size(), &scales[static_cast<size_t>(2 * ex)]) != 0) return -1;
        }
        return 0;
    };
    for (int l = 0; l < p->n_layers; ++l)
        if (load_layer(l, "layers." + std::to_string(l) + ".", p->attention[static_cast<size_t>(l)]) != 0) return -1;
    if (gv::model_of(g).has_mtp) {   // the MTP layer (model.cpp:175-191): its decoder layer, fc and norms, the draft head
        GV_REQUIRE(p->mtp, "gv_model_load_pack: the model has an MTP layer and the pack none");
        if (load_layer(p->n_layers, "mtp.layers.0.", true) != 0) return -1;
        if (get("mtp.fc.weight", T_Q4, H, 2 * H, t) != 0 || adopt(GV_MTP_FC, 0, 0, buf.data(), buf.size(), &t->global) != 0)
            return -1;
        for (const auto &[name, kind] : {std::make_pair("mtp.norm.weight", GV_MTP_NORM),
                                         std::make_pair("mtp.pre_fc_norm_embedding.weight", GV_MTP_PRE_E),
                                         std::make_pair("mtp.pre_fc_norm_hidden.weight", GV_MTP_PRE_H)})
            if (get_f32(name, H, t) != 0 || adopt(kind, 0, 0, buf.data(), buf.size(), nullptr) != 0) return -1;
        // draft_vocab.bin (model.cpp:806-811): int32 token ids, those outside the vocabulary skipped
        std::vector<int32_t> ids;
        if (std::FILE *f = std::fopen((p->dir + "/draft_vocab.bin").c_str(), "rb")) {
            int32_t id;
            while (std::fread(&id, 4, 1, f) == 1)
                if (id >= 0 && id < p->vocab) ids.push_back(id);
            std::fclose(f);
        }
        if (gv_model_set_draft_vocab(g, ids.data(), static_cast<int>(ids.size())) != 0) return -1;
    }
    return gv_model_set_position(g, 0);
}

}  // extern "C"
