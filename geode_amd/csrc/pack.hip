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
// Host code only: a JSON reader (RFC 8259, parsed into a flat tape), the staged manifest checks, the table and the
// file reads; the bytes go to the device through gv_model_adopt. The architectures read are qwen35moe (the GPU
// model's) and qwen35 (dense; its table is readable, the GPU model refuses it).
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

// ---------------------------------------------------------------- JSON (RFC 8259), read into a flat tape
// The document is parsed once, without recursion, into `nodes` in document order: a scalar is one node; an array or
// an object is a node whose `skip` is the index one past its last descendant, so its children are reached by jumping
// from one child to the next child's index. An object's children come in pairs, a key (a string node) then its value.
// Strings are decoded (escapes, UTF-16 surrogate pairs to UTF-8) into one byte arena; numbers follow the RFC's
// grammar exactly and are converted with strtod. Lookups walk a container's children (manifests are small).
class JsonTape {
public:
    enum Kind : uint8_t { kNull, kTrue, kFalse, kNumber, kString, kArray, kObject };
    struct Node {
        Kind kind;
        uint32_t skip;     // containers: one past the last descendant; scalars: own index + 1
        uint32_t off, len; // strings: the decoded bytes in the arena
        double number;
    };

    // a position in the tape; an absent member or element is the null view (kind() == kNull, valid() false)
    class View {
    public:
        View() = default;
        View(const JsonTape *t, uint32_t i) : t_(t), i_(i) {}
        bool valid() const { return t_ != nullptr; }
        Kind kind() const { return t_ ? t_->nodes_[i_].kind : kNull; }
        bool is(Kind k) const { return kind() == k; }
        // members and elements
        View member(const char *key) const {
            if (!is(kObject)) return {};
            const size_t kl = std::strlen(key);
            for (uint32_t c = i_ + 1; c < node().skip; c = t_->nodes_[c + 1].skip)
                if (t_->nodes_[c].len == kl && std::memcmp(t_->arena_.data() + t_->nodes_[c].off, key, kl) == 0)
                    return View(t_, c + 1);
            return {};
        }
        View operator[](const char *key) const { return member(key); }
        size_t count() const {
            if (!is(kArray) && !is(kObject)) return 0;
            size_t n = 0;
            for (uint32_t c = i_ + 1; c < node().skip; c = t_->nodes_[c].skip) ++n;
            return is(kObject) ? n / 2 : n;
        }
        View element(size_t k) const {
            if (!is(kArray)) return {};
            uint32_t c = i_ + 1;
            for (size_t j = 0; j < k && c < node().skip; ++j) c = t_->nodes_[c].skip;
            return c < node().skip ? View(t_, c) : View();
        }
        template <typename F> void each_member(F &&f) const {   // f(key, value)
            if (!is(kObject)) return;
            for (uint32_t c = i_ + 1; c < node().skip; c = t_->nodes_[c + 1].skip)
                f(std::string(t_->arena_.data() + t_->nodes_[c].off, t_->nodes_[c].len), View(t_, c + 1));
        }
        // scalars
        std::string text(const char *fallback = "") const {
            return is(kString) ? std::string(t_->arena_.data() + node().off, node().len) : std::string(fallback);
        }
        double number(double fallback) const { return is(kNumber) ? node().number : fallback; }
        // an integral number in [lo, hi] (false: absent, not a number, fractional or out of range)
        bool integer(int64_t lo, int64_t hi, int64_t &out) const {
            if (!is(kNumber)) return false;
            const double v = node().number;
            if (!(v >= static_cast<double>(lo) && v <= static_cast<double>(hi)) || v != std::floor(v)) return false;
            out = static_cast<int64_t>(v);
            return true;
        }
        bool flag() const { return is(kTrue); }

    private:
        const Node &node() const { return t_->nodes_[i_]; }
        const JsonTape *t_ = nullptr;
        uint32_t i_ = 0;
    };

    View root() const { return nodes_.empty() ? View() : View(this, 0); }

    // false with a message naming the byte offset and what was wrong
    bool parse(const char *text, size_t n, std::string &err) {
        nodes_.clear();
        arena_.clear();
        s_ = text;
        e_ = text + n;
        p_ = text;
        std::vector<uint32_t> open;   // indices of the containers not yet closed
        bool want_value = true;       // a value may (must) come next
        for (;;) {
            blanks();
            if (want_value) {
                if (p_ == e_) return bad("the text ends where a value is expected", err);
                const char c = *p_;
                if (c == ']' && !open.empty() && nodes_[open.back()].kind == kArray &&
                    nodes_.size() == open.back() + size_t{1}) {   // an empty array (no element pushed yet)
                    ++p_;
                    close(open);
                    want_value = false;
                } else if (c == '[' || c == '{') {
                    ++p_;
                    open.push_back(push(c == '[' ? kArray : kObject));
                    blanks();
                    if (c == '{') {
                        if (p_ < e_ && *p_ == '}') {
                            ++p_;
                            close(open);
                            want_value = false;
                        } else if (!key(err)) {
                            return false;
                        }
                    }
                    // an array: its first value (or ']') comes next; want_value stays true
                } else {
                    if (!scalar(err)) return false;
                    want_value = false;
                }
                if (!want_value && open.empty()) break;
                continue;
            }
            // after a value: a separator or the end of the enclosing container
            if (p_ == e_) return bad("the text ends inside an array or object", err);
            const Kind in = nodes_[open.back()].kind;
            const char c = *p_++;
            if (c == ',') {
                blanks();
                if (in == kObject && !key(err)) return false;
                want_value = true;
            } else if ((c == ']' && in == kArray) || (c == '}' && in == kObject)) {
                close(open);
                if (open.empty()) break;
            } else {
                --p_;
                return bad(in == kArray ? "',' or ']' expected after an array element"
                                        : "',' or '}' expected after an object member", err);
            }
        }
        blanks();
        if (p_ != e_) return bad("more text after the document's value", err);
        return true;
    }

private:
    uint32_t push(Kind k) {
        const uint32_t i = static_cast<uint32_t>(nodes_.size());
        nodes_.push_back(Node{k, i + 1, 0, 0, 0.0});
        return i;
    }
    void close(std::vector<uint32_t> &open) {
        nodes_[open.back()].skip = static_cast<uint32_t>(nodes_.size());
        open.pop_back();
    }
    void blanks() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool bad(const char *what, std::string &err) {
        err = std::string(what) + " (byte " + std::to_string(p_ - s_) + ")";
        return false;
    }
    // an object member's key and the ':' after it
    bool key(std::string &err) {
        if (p_ == e_ || *p_ != '"') return bad("an object member must start with a quoted key", err);
        if (!string_node(err)) return false;
        blanks();
        if (p_ == e_ || *p_ != ':') return bad("':' expected after an object key", err);
        ++p_;
        return true;
    }
    bool scalar(std::string &err) {
        const char c = *p_;
        if (c == '"') return string_node(err);
        if (c == '-' || (c >= '0' && c <= '9')) return number_node(err);
        static const struct { const char *word; Kind kind; } words[] = {{"null", kNull}, {"true", kTrue}, {"false", kFalse}};
        for (const auto &w : words) {
            const size_t wl = std::strlen(w.word);
            if (static_cast<size_t>(e_ - p_) >= wl && std::memcmp(p_, w.word, wl) == 0) {
                p_ += wl;
                push(w.kind);
                return true;
            }
        }
        return bad("a value is expected (object, array, string, number, true, false or null)", err);
    }
    // RFC 8259 section 6: -? (0 | [1-9][0-9]*) (. [0-9]+)? ([eE] [+-]? [0-9]+)?
    bool number_node(std::string &err) {
        const char *b = p_;
        auto digits = [&] {
            const char *d = p_;
            while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
            return p_ > d;
        };
        if (*p_ == '-') ++p_;
        if (p_ < e_ && *p_ == '0') ++p_;
        else if (!digits()) return bad("a number needs a digit after its sign", err);
        if (p_ < e_ && *p_ == '.') {
            ++p_;
            if (!digits()) return bad("a number needs digits after its decimal point", err);
        }
        if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
            ++p_;
            if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
            if (!digits()) return bad("a number needs digits in its exponent", err);
        }
        char buf[64];
        const size_t n = static_cast<size_t>(p_ - b);
        if (n >= sizeof buf) return bad("a number longer than 63 characters", err);
        std::memcpy(buf, b, n);
        buf[n] = '\0';
        const uint32_t i = push(kNumber);
        nodes_[i].number = std::strtod(buf, nullptr);
        return true;
    }
    static int hexval(char c) {
        return c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
    }
    bool unit16(uint32_t &u) {   // the four hex digits of a \u escape, p_ past the 'u'
        if (e_ - p_ < 4) return false;
        u = 0;
        for (int k = 0; k < 4; ++k) {
            const int h = hexval(p_[k]);
            if (h < 0) return false;
            u = u * 16 + static_cast<uint32_t>(h);
        }
        p_ += 4;
        return true;
    }
    void put_code_point(uint32_t cp) {   // UTF-8: 1 to 4 bytes
        char b[4];
        int n;
        if (cp < 0x80) {
            b[0] = static_cast<char>(cp);
            n = 1;
        } else {
            n = cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
            for (int k = n - 1; k > 0; --k, cp >>= 6) b[k] = static_cast<char>(0x80 | (cp & 0x3F));
            static const uint8_t lead[5] = {0, 0, 0xC0, 0xE0, 0xF0};
            b[0] = static_cast<char>(lead[n] | cp);
        }
        arena_.append(b, static_cast<size_t>(n));
    }
    bool string_node(std::string &err) {
        ++p_;   // the opening quote
        const uint32_t i = push(kString);
        nodes_[i].off = static_cast<uint32_t>(arena_.size());
        for (;;) {
            const char *run = p_;   // a run of plain bytes copied at once
            while (p_ < e_ && *p_ != '"' && *p_ != '\\' && static_cast<unsigned char>(*p_) >= 0x20) ++p_;
            arena_.append(run, static_cast<size_t>(p_ - run));
            if (p_ == e_) return bad("a string is not closed", err);
            if (*p_ == '"') break;
            if (*p_ != '\\') return bad("a control byte inside a string must be escaped", err);
            if (++p_ == e_) return bad("a string ends inside an escape", err);
            const char esc = *p_++;
            const char *plain = std::strchr("\"\\/bfnrt", esc);
            if (esc != '\0' && plain) {
                static const char decoded[] = "\"\\/\b\f\n\r\t";
                arena_.push_back(decoded[plain - "\"\\/bfnrt"]);
                continue;
            }
            if (esc != 'u') return bad("an unknown escape in a string", err);
            uint32_t u;
            if (!unit16(u)) return bad("\\u needs four hex digits", err);
            if (u >= 0xDC00 && u <= 0xDFFF) return bad("a low surrogate without its high surrogate", err);
            if (u >= 0xD800 && u <= 0xDBFF) {   // a pair: the low surrogate must follow as \uDC00..\uDFFF
                uint32_t lo;
                if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return bad("a high surrogate without its pair", err);
                p_ += 2;
                if (!unit16(lo) || lo < 0xDC00 || lo > 0xDFFF) return bad("a high surrogate without its pair", err);
                u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
            }
            put_code_point(u);
        }
        ++p_;   // the closing quote
        nodes_[i].len = static_cast<uint32_t>(arena_.size()) - nodes_[i].off;
        return true;
    }

    std::vector<Node> nodes_;
    std::string arena_;
    const char *s_ = nullptr, *e_ = nullptr, *p_ = nullptr;
};
using JView = JsonTape::View;

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
    JsonTape doc;        // geode.json
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

// Opening a pack: the manifest is read into gv_pack in stages, each checking what the later stages and the loads rely
// on, and a refusal names the entry at fault. What is checked follows Pack::open (pack.cpp:39-308) — the format and
// version, the architecture, every listed file present at its listed size (an optional one may be absent: its tensors
// are then skipped), the geometry, each tensor's type, shape and byte extent inside its file, dense.bin in use, the
// embedding, the expert table covering every layer with its scales, q3's bit order — but dense.bin is not read into
// memory: the tensors are read from their files when a model adopts them. Integers in the manifest must be integral
// JSON numbers in range; a tensor's dimensions are at most 2^32 and its element count at most 2^48 (byte counts stay
// far inside 64 bits).
class PackOpener {
public:
    PackOpener(gv_pack &P, std::string &err) : P_(P), err_(err) {}

    bool run(const std::string &dir) {
        P_.dir = dir;
        return read_manifest() && check_format() && check_files() && read_geometry() && read_tensors() &&
               read_expert_table() && read_formats();
    }

private:
    static constexpr int64_t kMaxDim = int64_t{1} << 32;
    static constexpr int64_t kMaxElements = int64_t{1} << 48;

    bool refuse(const std::string &why) {
        err_ = why;
        return false;
    }
    static std::string number_text(double v) {
        char b[32];
        std::snprintf(b, sizeof b, "%g", v);
        return b;
    }
    JView manifest() const { return P_.doc.root(); }

    bool read_manifest() {
        const std::string path = P_.dir + "/geode.json";
        uint64_t size = 0;
        ReadFile f;
        if (!file_size(path, size) || !f.open(path)) return refuse("cannot read " + path);
        std::string text(static_cast<size_t>(size), '\0');
        if (size && !f.read(0, text.data(), text.size())) return refuse("cannot read " + path);
        const uint64_t h = fnv(text.data(), text.size());   // the pack print a state file carries (state.cpp:227-238)
        P_.print = h ? h : 1;
        std::string why;
        if (!P_.doc.parse(text.data(), text.size(), why)) return refuse("geode.json is not valid JSON: " + why);
        if (!manifest().is(JsonTape::kObject)) return refuse("geode.json must hold a JSON object");
        return true;
    }

    bool check_format() {
        const JView m = manifest();
        int64_t version = 0;
        if (m["format"].text() != "geode-pack" || !m["version"].integer(1, 1, version))
            return refuse("geode.json describes format '" + m["format"].text("(none)") + "' version " +
                          (m["version"].is(JsonTape::kNumber) ? number_text(m["version"].number(0)) : "(none)") +
                          "; this reader takes geode-pack version 1");
        P_.arch = m["arch"].text();
        if (P_.arch != "qwen35moe" && P_.arch != "qwen35")
            return refuse("architecture '" + P_.arch + "' is not one this library loads (qwen35moe, qwen35)");
        P_.dense = P_.arch == "qwen35";
        return true;
    }

    bool check_files() {
        const JView list = manifest()["files"];
        for (size_t k = 0; k < list.count(); ++k) {
            const JView entry = list.element(k);
            const std::string name = entry["name"].text();
            int64_t listed = 0;
            if (name.empty() || !entry["size"].integer(0, INT64_MAX, listed))
                return refuse("geode.json files[" + std::to_string(k) + "] needs a name and a byte size");
            uint64_t have = 0;
            if (!file_size(P_.dir + "/" + name, have)) {
                if (entry["optional"].flag()) {
                    absent_.push_back(name);
                    continue;
                }
                return refuse(name + " is listed in geode.json but missing from " + P_.dir);
            }
            if (have != static_cast<uint64_t>(listed))
                return refuse(name + " holds " + std::to_string(have) + " bytes; geode.json lists " + std::to_string(listed));
            P_.files.push_back(name);
            P_.sizes.push_back(have);
        }
        return true;
    }

    // an optional integer of the config (absent: 0), refused when present but not an integer in [0, 2^31)
    bool config_int(const char *key, int &out) {
        const JView v = manifest()["config"][key];
        int64_t x = 0;
        if (v.valid() && !v.integer(0, INT32_MAX, x)) return refuse(std::string("config.") + key + " is not a count");
        out = static_cast<int>(x);
        return true;
    }

    bool read_geometry() {
        const JView c = manifest()["config"];
        gv_pack &P = P_;
        const char *ff_key = P.dense ? "intermediate_size" : "shared_expert_intermediate_size";
        const std::pair<const char *, int *> ints[] = {
            {"hidden_size", &P.hidden}, {"num_hidden_layers", &P.n_layers}, {"vocab_size", &P.vocab},
            {"num_attention_heads", &P.n_heads}, {"num_key_value_heads", &P.n_kv_heads}, {"head_dim", &P.head_dim},
            {"linear_num_key_heads", &P.gdn_k_heads}, {"linear_num_value_heads", &P.gdn_v_heads},
            {"linear_key_head_dim", &P.gdn_k_dim}, {"linear_value_head_dim", &P.gdn_v_dim},
            {"linear_conv_kernel_dim", &P.conv_kernel}, {"num_experts", &P.n_experts},
            {"num_experts_per_tok", &P.top_k}, {"moe_intermediate_size", &P.moe_ff}, {ff_key, &P.shared_ff}};
        for (const auto &[key, dst] : ints)
            if (!config_int(key, *dst)) return false;
        P.eps = static_cast<float>(c["rms_norm_eps"].number(1e-6));
        const JView rope = c["rope_parameters"];
        P.rope_theta = static_cast<float>(rope["rope_theta"].number(10000.0));
        P.rope_dim = static_cast<int>(P.head_dim * rope["partial_rotary_factor"].number(1.0));
        const std::string g = "model geometry: ";
        if (P.n_layers < 1 || P.n_layers > 1024) return refuse(g + "num_hidden_layers must be 1..1024");
        const JView types = c["layer_types"];
        if (types.count() != static_cast<size_t>(P.n_layers))
            return refuse(g + "config.layer_types lists " + std::to_string(types.count()) + " layers for num_hidden_layers " +
                          std::to_string(P.n_layers));
        P.attention.clear();
        for (int l = 0; l < P.n_layers; ++l)
            P.attention.push_back(types.element(static_cast<size_t>(l)).text() == "full_attention");
        if (P.hidden <= 0 || P.hidden % 16)
            return refuse(g + "hidden_size " + std::to_string(P.hidden) + " is not a positive multiple of 16");
        if (P.dense && (P.n_experts != 0 || P.shared_ff <= 0 || P.shared_ff % 16))
            return refuse(g + "a dense model needs no experts and an intermediate_size that is a multiple of 16");
        if (!P.dense && (P.top_k < 1 || P.top_k > P.n_experts))
            return refuse(g + "num_experts_per_tok must be 1..num_experts");
        if (P.gdn_v_heads % std::max(1, P.gdn_k_heads))
            return refuse(g + "linear_num_value_heads is not a multiple of linear_num_key_heads");
        if (P.n_heads % std::max(1, P.n_kv_heads))
            return refuse(g + "num_attention_heads is not a multiple of num_key_value_heads");
        if (P.rope_dim % 2) return refuse(g + "the rotary dimensions are odd");
        return true;
    }

    // a tensor's entry; false with the refusal set; skip set when its file is an absent optional one
    bool tensor_entry(const std::string &name, const JView &e, Tensor &x, bool &skip) {
        const std::string file = e["file"].text();
        skip = std::find(absent_.begin(), absent_.end(), file) != absent_.end();
        if (skip) return true;
        const std::string at = "tensor " + name + ": ";
        x.type = type_of(e["type"].text());
        if (x.type == T_UNKNOWN) return refuse(at + "type '" + e["type"].text() + "' is not a known tensor type");
        const JView shape = e["shape"];
        int64_t elements = 1, offset = 0;
        bool in_range = e["offset"].integer(0, kMaxElements, offset);
        for (size_t i = 0; i < shape.count() && in_range; ++i) {
            int64_t d = 0;
            in_range = shape.element(i).integer(1, kMaxDim, d) && elements <= kMaxElements / d;
            elements *= d;
            x.shape.push_back(d);
        }
        if (!in_range) return refuse(at + "its shape or offset is outside what a pack can hold");
        // rows and columns: [d0, d1 x d2 x ...]; a vector is one row; no dimension at all, one value
        x.rows = x.shape.size() >= 2 ? x.shape[0] : 1;
        x.cols = x.shape.empty() ? 1 : elements / x.rows;
        x.file = P_.file_index(file);
        if (x.file < 0) return refuse(at + "file '" + file + "' is not one of geode.json's files");
        x.offset = static_cast<uint64_t>(offset);
        x.global = static_cast<float>(e["global"].number(1.0));
        if (quantized(x.type) && x.cols % 16)
            return refuse(at + "a quantized tensor needs a multiple of 16 columns (it has " + std::to_string(x.cols) + ")");
        const uint64_t fsize = P_.sizes[static_cast<size_t>(x.file)];
        if (x.offset > fsize || x.bytes() > fsize - x.offset) return refuse(at + "its bytes run past the end of " + file);
        return true;
    }

    bool read_tensors() {
        const JView table = manifest()["tensors"];
        if (!table.is(JsonTape::kObject)) return refuse("geode.json has no tensor table (\"tensors\")");
        bool ok = true, in_dense = false;
        table.each_member([&](const std::string &name, const JView &e) {
            if (!ok) return;
            Tensor x;
            bool skip = false;
            ok = tensor_entry(name, e, x, skip);
            if (!ok || skip) return;
            in_dense = in_dense || P_.files[static_cast<size_t>(x.file)] == "dense.bin";
            P_.tensors[name] = std::move(x);
        });
        if (!ok) return false;
        if (!in_dense) return refuse("geode.json places no tensor in dense.bin");
        const Tensor *embed = P_.find("embed_tokens.weight");
        if (!embed || !quantized(embed->type) || embed->cols != P_.hidden)
            return refuse("embed_tokens.weight must be a quantized [vocab, hidden_size] tensor");
        return true;
    }

    // expert layer l's entry (l = n_layers: the MTP layer's) and its scales tensor
    bool expert_layer(const JView &e, int l) {
        const std::string at = "experts, layer " + std::to_string(l) + ": ";
        ExpertLayer x;
        x.file = P_.file_index(e["file"].text());
        if (x.file < 0) return refuse(at + "file '" + e["file"].text() + "' is not one of geode.json's files");
        int64_t v = 0;
        if (e["stride"].is(JsonTape::kNumber)) {   // one format, expert i at offset + i x stride
            if (!e["offset"].integer(0, kMaxElements, v)) return refuse(at + "the offset is not a byte position");
            x.offset = static_cast<uint64_t>(v);
            if (!e["stride"].integer(0, kMaxElements, v)) return refuse(at + "the stride is not a byte count");
            x.stride = static_cast<uint64_t>(v);
            x.type = type_of(e["format"].text());
        } else {                                   // per-expert offsets and formats
            const JView offs = e["offsets"], fmts = e["formats"];
            if (offs.count() != static_cast<size_t>(P_.n_experts) || fmts.count() != offs.count())
                return refuse(at + std::to_string(offs.count()) + " experts listed, config.num_experts is " +
                              std::to_string(P_.n_experts));
            for (size_t i = 0; i < offs.count(); ++i) {
                if (!offs.element(i).integer(0, kMaxElements, v)) return refuse(at + "an offset is not a byte position");
                x.offsets.push_back(static_cast<uint64_t>(v));
                x.types.push_back(type_of(fmts.element(i).text()));
            }
        }
        P_.experts.push_back(std::move(x));
        const std::string scales = l < P_.n_layers ? "layers." + std::to_string(l) + ".mlp.experts.scales"
                                                   : "mtp.layers.0.mlp.experts.scales";
        const Tensor *s = P_.find(scales);
        if (!s || s->type != T_F32 || s->rows != P_.n_experts || s->cols != 2)
            return refuse(at + "the scales tensor " + scales + " is missing or not f32 [num_experts, 2]");
        return true;
    }

    bool read_expert_table() {
        const JView layers = manifest()["experts"]["layers"];
        const size_t want = P_.dense ? 0 : static_cast<size_t>(P_.n_layers);
        if (layers.count() != want)
            return refuse("geode.json's expert table has " + std::to_string(layers.count()) + " layers; the model has " +
                          std::to_string(want) + " MoE layers");
        for (size_t l = 0; l < want; ++l)
            if (!expert_layer(layers.element(l), static_cast<int>(l))) return false;
        const JView mtp = manifest()["mtp"];
        if (mtp.is(JsonTape::kObject)) {
            if (!P_.dense && !expert_layer(mtp["experts"], P_.n_layers)) return false;
            P_.mtp = true;
        }
        return true;
    }

    bool read_formats() {
        const JView formats = manifest()["formats"];
        bool q3 = false;
        for (const auto &kv : P_.tensors) q3 = q3 || kv.second.type == T_Q3;
        for (const auto &x : P_.experts) {
            q3 = q3 || x.type == T_Q3;
            q3 = q3 || std::find(x.types.begin(), x.types.end(), static_cast<int>(T_Q3)) != x.types.end();
        }
        // q3 packs written before the values' high bits went in value order are not readable (kernels.hpp's q3)
        if (q3 && formats["q3"]["high_bits"].text() != "value order")
            return refuse("q3 tensors need formats.q3.high_bits = \"value order\"");
        P_.tile8 = formats["q4"]["layout"].text() == "tile8";
        return true;
    }

    gv_pack &P_;
    std::string &err_;
    std::vector<std::string> absent_;   // optional files not present
};

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
    if (!PackOpener(*P, e).run(dir)) {
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
