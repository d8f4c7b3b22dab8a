// oracle_core.cpp - the q4 format, the products, RMSNorm and routing, restated from the reference on the CPU.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP path, never part of it.
//
// Pinning (what checks each function; tests/test_oracle_*.py):
//   e4m3_value         all 256 bytes against the reference built from its sources (oracle/_ref) and the OCP E4M3FN
//                      closed form
//   e4m3_byte          oracle/_ref on every E4M3 midpoint, the values themselves and random floats; monotonicity
//   q4_block / pack    oracle/_ref bit for bit on seeded blocks (golden fixtures); invariant: no candidate scale
//                      gives a smaller squared error
//   dequant_rows       oracle/_ref; closed form kQ4[c] * e4m3 * global exhaustively over codes x scale bytes
//   matvec_rows        oracle/_ref bit for bit; fp64 brute force within fp32 rounding
//   quantize_activation, matvec_rows_q
//                      oracle/_ref bit for bit; integer block sums against brute force
//   matvec_bf16        oracle/_ref bit for bit (matvec_rows_bf16_multi); fp64 brute force
//   rmsnorm            oracle/_ref bit for bit; closed form in fp64
//   route_topk         brute force (a full sort by probability, ties to the lower index), weights summing to 1;
//                      not compilable alone (it sits in model.cpp): parity pinned by brute force only
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <numeric>
#include <thread>
#include <vector>

#include "oracle_internal.hpp"

namespace orc {

// ---------------------------------------------------------------- generator
uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// ---------------------------------------------------------------- fp16 / bf16
uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return static_cast<uint16_t>(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);   // rounds to infinity
    const int e = static_cast<int>(ax >> 23);
    if (e < 113) {   // below 2^-14: a subnormal half, k * 2^-24
        if (e == 0) return static_cast<uint16_t>(sign);
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - e;   // k = m / 2^shift
        if (shift > 25) return static_cast<uint16_t>(sign);
        uint32_t k = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (k & 1u))) ++k;
        return static_cast<uint16_t>(sign | k);
    }
    uint32_t h = (static_cast<uint32_t>(e - 112) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return static_cast<uint16_t>(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {   // subnormal: m * 2^-24
            float v = std::ldexp(static_cast<float>(m), -24);
            std::memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u = u + 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// ---------------------------------------------------------------- threads
// A persistent pool: parallel_for(items, chunk, fn) splits [0, items) in chunks taken dynamically
// (threads.cpp:313's dynamic split; the reference's matmul uses chunks of 16 rows, model.cpp:3358-3360).
class Pool {
public:
    explicit Pool(int n) { resize(n); }
    ~Pool() { stop(); }
    int size() const { return static_cast<int>(workers_.size()) + 1; }
    void resize(int n) {
        stop();
        quit_ = false;
        for (int i = 1; i < n; ++i) workers_.emplace_back([this] { loop(); });
    }
    // One caller at a time uses the workers; a caller that finds them busy (another host thread's call, or a call
    // from inside a task) runs its whole range itself, so concurrent callers never share the pool's state.
    void run(int64_t items, int64_t chunk, const std::function<void(int64_t, int64_t)> &fn) {
        if (items <= 0) return;
        std::unique_lock<std::mutex> own(busy_, std::try_to_lock);
        if (!own.owns_lock() || workers_.empty() || items <= chunk) {
            fn(0, items);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            fn_ = &fn;
            items_ = items;
            chunk_ = chunk;
            next_.store(0);
            active_ = static_cast<int>(workers_.size());
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return active_ == 0; });
        fn_ = nullptr;
    }

private:
    void work() {
        for (;;) {
            const int64_t a = next_.fetch_add(chunk_);
            if (a >= items_) break;
            (*fn_)(a, std::min(items_, a + chunk_));
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return quit_ || gen_ != seen; });
                if (quit_) return;
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> lk(mu_);
            if (--active_ == 0) done_cv_.notify_all();
        }
    }
    void stop() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            quit_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
        workers_.clear();
    }
    std::vector<std::thread> workers_;
    std::mutex busy_;   // held by the caller whose range the workers are on
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int64_t, int64_t)> *fn_ = nullptr;
    int64_t items_ = 0, chunk_ = 1;
    std::atomic<int64_t> next_{0};
    int active_ = 0;
    uint64_t gen_ = 0;
    bool quit_ = false;
};

Pool &pool() {
    static Pool p(1);
    return p;
}

void par(int64_t items, int64_t chunk, const std::function<void(int64_t, int64_t)> &fn) {
    pool().run(items, chunk, fn);
}

// ---------------------------------------------------------------- q4
// kQ4: the integer levels in code order (kernels.cpp:30)
constexpr int8_t kQ4[16] = {1, 3, 5, 7, 9, 11, 13, 15, -1, -3, -5, -7, -9, -11, -13, -15};

const float *e4m3_table() {
    static const std::vector<float> t = [] {
        std::vector<float> v(256);
        for (int b = 0; b < 256; ++b) {
            const int sign = b >> 7, ex = (b >> 3) & 15, man = b & 7;
            float x = ex == 0 ? std::ldexp(static_cast<float>(man) / 8.0f, -6)
                              : std::ldexp(1.0f + static_cast<float>(man) / 8.0f, ex - 7);
            if (ex == 15 && man == 7) x = std::numeric_limits<float>::quiet_NaN();
            v[static_cast<size_t>(b)] = sign ? -x : x;
        }
        return v;
    }();
    return t.data();
}

uint8_t e4m3_byte(float x) {
    const float *v = e4m3_table();   // codes 0x00..0x7E increase
    if (!(x > 0.0f)) return 0;
    if (x >= v[126]) return 126;
    const int hi = static_cast<int>(std::upper_bound(v, v + 127, x) - v);   // v[hi] > x
    const int lo = hi - 1;
    const float dl = x - v[lo], dh = v[hi] - x;
    if (dl < dh) return static_cast<uint8_t>(lo);
    if (dh < dl) return static_cast<uint8_t>(hi);
    return static_cast<uint8_t>(lo % 2 == 0 ? lo : hi);
}

void q4_block(const float *x, float s2, uint8_t &scale_byte, uint8_t codes[16]) {
    float amax = 0.0f;
    for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[i]));
    int cand[10], nc = 0;
    for (const float t : {15.0f, 13.0f}) {
        const int b0 = e4m3_byte(amax / (t * s2));
        for (int k = -2; k <= 2; ++k) cand[nc++] = std::clamp(b0 + k, 0, 0x7E);
    }
    float best = std::numeric_limits<float>::infinity();
    uint8_t tmp[16];
    const float *e4 = e4m3_table();
    for (int c = 0; c < nc; ++c) {
        const float scale = e4[cand[c]] * s2, safe = scale == 0.0f ? 1.0f : scale;
        float err = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const float y = x[i] / safe, a = std::min(std::fabs(y), 15.0f);
            const int idx = std::clamp(static_cast<int>(std::nearbyint((a - 1.0f) * 0.5f)), 0, 7);
            const bool neg = y < 0.0f;
            const float q = static_cast<float>(neg ? -(2 * idx + 1) : 2 * idx + 1) * scale;
            const float d = q - x[i];
            err += d * d;
            tmp[i] = static_cast<uint8_t>(idx + (neg ? 8 : 0));
        }
        if (err < best) {
            best = err;
            scale_byte = static_cast<uint8_t>(cand[c]);
            std::copy(tmp, tmp + 16, codes);
        }
    }
}

// the 16 levels of block b of a row (kernels.cpp:86-97, q4 case)
inline void block_levels(const uint8_t *row, int b, int8_t v[16]) {
    const uint8_t *c = row + b * 8;
    for (int j = 0; j < 8; ++j) {
        v[2 * j] = kQ4[c[j] & 15];
        v[2 * j + 1] = kQ4[c[j] >> 4];
    }
}

void matvec_exact(const uint8_t *w, int64_t cols, float global, const float *x, float *y, int64_t r0, int64_t r1) {
    const float *e4 = e4m3_table();
    const int nb = static_cast<int>(cols / 16);
    const size_t rb = static_cast<size_t>(nb) * 9;
    for (int64_t r = r0; r < r1; ++r) {
        const uint8_t *row = w + static_cast<size_t>(r) * rb;
        const uint8_t *sc = row + static_cast<size_t>(nb) * 8;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            int8_t v[16];
            block_levels(row, b, v);
            const float *xb = x + b * 16;
            float s = 0.0f;
            for (int i = 0; i < 16; ++i) s += static_cast<float>(v[i]) * xb[i];
            acc += s * e4[sc[b]];
        }
        y[r] = acc * global * 1.0f;
    }
}

void quantize(const float *x, int64_t cols, QAct &a) {
    const int64_t nb = cols / 16;
    a.q.resize(static_cast<size_t>(cols));
    a.scale.resize(static_cast<size_t>(nb));
    a.bsum.resize(static_cast<size_t>(nb));
    for (int64_t b = 0; b < nb; ++b) {
        const float *xb = x + b * 16;
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(xb[i]));
        const float s = amax / 127.0f, inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        a.scale[static_cast<size_t>(b)] = s;
        int32_t sum = 0;
        for (int i = 0; i < 16; ++i) {
            const auto q = static_cast<int8_t>(std::clamp(std::lrint(xb[i] * inv), -127L, 127L));
            a.q[static_cast<size_t>(b * 16 + i)] = q;
            sum += q;
        }
        a.bsum[static_cast<size_t>(b)] = sum;
    }
}

void matvec_q(const uint8_t *w, int64_t cols, float global, const QAct &a, float *y, int64_t r0, int64_t r1) {
    const float *e4 = e4m3_table();
    const int nb = static_cast<int>(cols / 16);
    const size_t rb = static_cast<size_t>(nb) * 9;
    for (int64_t r = r0; r < r1; ++r) {
        const uint8_t *row = w + static_cast<size_t>(r) * rb;
        const uint8_t *sc = row + static_cast<size_t>(nb) * 8;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            int8_t v[16];
            block_levels(row, b, v);
            int32_t s = 0;
            for (int i = 0; i < 16; ++i) s += v[i] * a.q[static_cast<size_t>(b * 16 + i)];
            acc += static_cast<float>(s) * (e4[sc[b]] * a.scale[static_cast<size_t>(b)]);
        }
        y[r] = acc * global * 1.0f;
    }
}

void bf16_rows(const uint16_t *w, int64_t cols, int n, const float *const *xs, float *const *ys, int64_t r0,
               int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
        const uint16_t *row = w + static_cast<size_t>(r) * cols;
        for (int t = 0; t < n; ++t) {
            float acc[8] = {};
            const float *x = xs[t];
            for (int64_t c = 0; c < cols; c += 8)
                for (int j = 0; j < 8; ++j) acc[j] += bf16_to_f32(row[c + j]) * x[c + j];
            ys[t][r] = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
        }
    }
}

void rmsnorm(const float *x, const float *w, float *out, int n, float eps, bool zero_centered) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += static_cast<double>(x[i]) * x[i];
    const float inv = 1.0f / std::sqrt(static_cast<float>(ss / n) + eps);
    if (!w) {
        for (int i = 0; i < n; ++i) out[i] = x[i] * inv;
        return;
    }
    for (int i = 0; i < n; ++i) out[i] = x[i] * inv * (zero_centered ? 1.0f + w[i] : w[i]);
}

void route_topk(const float *logits, int E, int K, int *ids, float *weights) {
    std::vector<float> p(logits, logits + E);
    const float mx = *std::max_element(p.begin(), p.end());
    float sum = 0.0f;
    for (float &v : p) sum += (v = std::exp(v - mx));
    for (float &v : p) v /= sum;
    std::vector<int> order(static_cast<size_t>(E));
    std::iota(order.begin(), order.end(), 0);
    // the reference's partial_sort leaves equal probabilities in an unspecified order; the build sends them to the
    // lower index (as the reference's GPU route kernel, gpu8_kernels.inc:974-978)
    std::partial_sort(order.begin(), order.begin() + K, order.end(), [&](int a, int b) {
        const float x = p[static_cast<size_t>(a)], y = p[static_cast<size_t>(b)];
        return x > y || (x == y && a < b);
    });
    float top = 0.0f;
    for (int i = 0; i < K; ++i) top += p[static_cast<size_t>(order[static_cast<size_t>(i)])];
    for (int i = 0; i < K; ++i) {
        ids[i] = order[static_cast<size_t>(i)];
        if (weights) weights[i] = p[static_cast<size_t>(order[static_cast<size_t>(i)])] / top;
    }
}

// ys[t] = W xs[t] for n tokens, the rows split over the pool in chunks of 16 (Model::matmul, model.cpp:3336-3491):
// mode 0 quantizes each token's activations first (the int8 path), mode 1 is the exact path
void matmul(const uint8_t *w, int64_t rows, int64_t cols, float global, int n, const float *const *xs,
            float *const *ys, int mode) {
    if (mode == 1) {
        par(rows, 16, [&](int64_t a, int64_t b) {
            for (int t = 0; t < n; ++t) matvec_exact(w, cols, global, xs[t], ys[t], a, b);
        });
        return;
    }
    std::vector<QAct> acts(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) quantize(xs[t], cols, acts[static_cast<size_t>(t)]);
    par(rows, 16, [&](int64_t a, int64_t b) {
        for (int t = 0; t < n; ++t) matvec_q(w, cols, global, acts[static_cast<size_t>(t)], ys[t], a, b);
    });
}

}  // namespace orc

using namespace orc;

extern "C" {

uint64_t orc_hash(uint64_t seed, uint64_t i) { return splitmix64(seed * 0xD1342543DE82EF95ull + i); }

void orc_fill_normal(uint64_t seed, int64_t n, float mean, float sigma, float *out) {
    const double two_pi = 6.283185307179586476925286766559;
    par(n, 4096, [&](int64_t a, int64_t b) {
        for (int64_t i = a; i < b; ++i) {
            const uint64_t k = static_cast<uint64_t>(i) >> 1;
            const double u1 = (static_cast<double>(orc_hash(seed, 2 * k) >> 11) + 0.5) * 0x1p-53;
            const double u2 = static_cast<double>(orc_hash(seed, 2 * k + 1) >> 11) * 0x1p-53;
            const double r = std::sqrt(-2.0 * std::log(u1));
            const double z = (i & 1) ? r * std::sin(two_pi * u2) : r * std::cos(two_pi * u2);
            out[i] = static_cast<float>(static_cast<double>(mean) + static_cast<double>(sigma) * z);
        }
    });
}

void orc_fill_uniform(uint64_t seed, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = (static_cast<float>(orc_hash(seed, static_cast<uint64_t>(i)) >> 40) + 0.5f) * 0x1p-24f;
}

uint16_t orc_f32_to_f16(float x) { return f32_to_f16(x); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_f32_to_bf16(float x) { return f32_to_bf16(x); }

void orc_set_threads(int n) { pool().resize(std::max(1, n)); }
int orc_threads(void) { return pool().size(); }

float orc_e4m3_value(uint8_t b) { return e4m3_table()[b]; }
uint8_t orc_e4m3_byte(float x) { return e4m3_byte(x); }
void orc_q4_block(const float *x, float s2, uint8_t *scale_byte, uint8_t *codes16) {
    q4_block(x, s2, *scale_byte, codes16);
}

float orc_q4_global(const float *w, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) m = std::max(m, std::fabs(w[i]));
    return m * 1.25f / (15.0f * 448.0f);
}

void orc_q4_pack(const float *w, int64_t rows, int64_t cols, float s2, uint8_t *out) {
    const int64_t nb = cols / 16;
    const size_t rb = static_cast<size_t>(nb) * 9;
    par(rows, 16, [&](int64_t a, int64_t b) {
        uint8_t codes[16];
        for (int64_t r = a; r < b; ++r) {
            uint8_t *o = out + static_cast<size_t>(r) * rb;
            for (int64_t blk = 0; blk < nb; ++blk) {
                uint8_t sb = 0;
                q4_block(w + r * cols + blk * 16, s2, sb, codes);
                for (int k = 0; k < 8; ++k) o[blk * 8 + k] = static_cast<uint8_t>(codes[2 * k] | (codes[2 * k + 1] << 4));
                o[cols / 2 + blk] = sb;
            }
        }
    });
}

void orc_dequant_rows(const uint8_t *w, int64_t rows, int64_t cols, float global, float *out) {
    const float *e4 = e4m3_table();
    const int nb = static_cast<int>(cols / 16);
    const size_t rb = static_cast<size_t>(nb) * 9;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t *row = w + static_cast<size_t>(r) * rb;
        const uint8_t *sc = row + static_cast<size_t>(nb) * 8;
        for (int b = 0; b < nb; ++b) {
            int8_t v[16];
            block_levels(row, b, v);
            const float s = e4[sc[b]] * global;
            for (int i = 0; i < 16; ++i) out[r * cols + b * 16 + i] = (static_cast<float>(v[i]) * 1.0f) * s;
        }
    }
}

void orc_matvec_rows(const uint8_t *w, int64_t rows, int64_t cols, float global, const float *x, float *y) {
    par(rows, 16, [&](int64_t a, int64_t b) { matvec_exact(w, cols, global, x, y, a, b); });
}

void orc_quantize_activation(const float *x, int64_t cols, int8_t *q, float *scale, int32_t *bsum) {
    QAct a;
    quantize(x, cols, a);
    std::memcpy(q, a.q.data(), static_cast<size_t>(cols));
    std::memcpy(scale, a.scale.data(), sizeof(float) * static_cast<size_t>(cols / 16));
    std::memcpy(bsum, a.bsum.data(), sizeof(int32_t) * static_cast<size_t>(cols / 16));
}

void orc_matvec_rows_q(const uint8_t *w, int64_t rows, int64_t cols, float global, const int8_t *q,
                       const float *scale, float *y) {
    QAct a;
    a.q.assign(q, q + cols);
    a.scale.assign(scale, scale + cols / 16);
    par(rows, 16, [&](int64_t r0, int64_t r1) { matvec_q(w, cols, global, a, y, r0, r1); });
}

void orc_matvec_bf16(const uint16_t *w, int64_t rows, int64_t cols, int n, const float *x, float *y) {
    std::vector<const float *> xs(static_cast<size_t>(n));
    std::vector<float *> ys(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) {
        xs[static_cast<size_t>(t)] = x + static_cast<size_t>(t) * cols;
        ys[static_cast<size_t>(t)] = y + static_cast<size_t>(t) * rows;
    }
    par(rows, 16, [&](int64_t a, int64_t b) { bf16_rows(w, cols, n, xs.data(), ys.data(), a, b); });
}

void orc_rmsnorm(const float *x, const float *w, float *out, int n, float eps, int zero_centered) {
    rmsnorm(x, w, out, n, eps, zero_centered != 0);
}

void orc_route_topk(const float *logits, int E, int K, int *ids, float *weights) {
    route_topk(logits, E, K, ids, weights);
}

}  // extern "C"
