// ref_shim.cpp - extern "C" entry points over the reference's own functions, compiled together with the reference
// sources where they lie (kernels.cpp, sampler.cpp, yue2_q4.cpp under /root/reference/engine/src) into
// oracle/_ref/libgeode_ref.so. Nothing of the reference is copied here: these wrappers only call it.
//
// TEST INFRASTRUCTURE ONLY: used to pin the oracle (tests/golden/make_golden.py writes its outputs as fixtures and
// tests/test_oracle_*.py compares against it when it is built). The product never loads it.
#include <cstdint>
#include <vector>

#include "kernels.hpp"
#include "sampler.hpp"
#include "yue2_q4.hpp"

using namespace geode;

namespace {
QView q4_view(const uint8_t *w, int64_t rows, int64_t cols, float global) {
    QView v;
    v.type = DType::Q4;
    v.rows = rows;
    v.cols = cols;
    v.row_bytes = row_bytes(DType::Q4, cols);
    v.data = w;
    v.global = global;
    return v;
}
}  // namespace

extern "C" {

__attribute__((visibility("default"))) float ref_e4m3_value(uint8_t b) { return e4m3_value(b); }

__attribute__((visibility("default"))) uint8_t ref_e4m3_byte(float x) { return yue2::e4m3_byte(x); }

__attribute__((visibility("default"))) void ref_q4_block(const float *x, float s2, uint8_t *scale, uint8_t *codes) {
    yue2::q4_block(x, s2, *scale, codes);
}

__attribute__((visibility("default"))) void ref_dequant_rows(const uint8_t *w, int64_t rows, int64_t cols,
                                                             float global, float *out) {
    const QView v = q4_view(w, rows, cols, global);
    for (int64_t r = 0; r < rows; ++r) dequant_row(v, r, out + r * cols);
}

__attribute__((visibility("default"))) void ref_matvec_rows(const uint8_t *w, int64_t rows, int64_t cols, float global,
                                                            const float *x, float *y) {
    matvec_rows(q4_view(w, rows, cols, global), x, y, 0, rows);
}

__attribute__((visibility("default"))) void ref_quantize_activation(const float *x, int64_t cols, int8_t *q,
                                                                    float *scale, int32_t *bsum) {
    QAct a;
    quantize_activation(x, cols, a);
    for (int64_t i = 0; i < cols; ++i) q[i] = a.q[static_cast<size_t>(i)];
    for (int64_t b = 0; b < cols / kBlock; ++b) {
        scale[b] = a.scale[static_cast<size_t>(b)];
        bsum[b] = a.bsum[static_cast<size_t>(b)];
    }
}

// the int8 path: x quantized by quantize_activation, then matvec_rows_q (matvec_rows_q_ref on x86)
__attribute__((visibility("default"))) void ref_matvec_rows_q(const uint8_t *w, int64_t rows, int64_t cols,
                                                              float global, const float *x, float *y) {
    QAct a;
    quantize_activation(x, cols, a);
    matvec_rows_q(q4_view(w, rows, cols, global), a, y, 0, rows);
}

__attribute__((visibility("default"))) void ref_matvec_bf16_multi(const uint16_t *w, int64_t rows, int64_t cols, int n,
                                                                  const float *x, float *y) {
    std::vector<const float *> xs(static_cast<size_t>(n));
    std::vector<float *> ys(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) {
        xs[static_cast<size_t>(t)] = x + static_cast<size_t>(t) * cols;
        ys[static_cast<size_t>(t)] = y + static_cast<size_t>(t) * rows;
    }
    matvec_rows_bf16_multi(w, cols, n, xs.data(), ys.data(), 0, rows);
}

__attribute__((visibility("default"))) void ref_rmsnorm(const float *x, const float *w, float *out, int n, float eps,
                                                        int zero_centered) {
    rmsnorm(x, w, out, n, eps, zero_centered != 0);
}

__attribute__((visibility("default"))) void ref_sample_seeded(const float *logits, int n, float temperature,
                                                              float top_p, int top_k, uint64_t seed, int draws,
                                                              int32_t *out) {
    Sampler s;
    s.seed(seed);
    SamplerParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    for (int d = 0; d < draws; ++d) out[d] = s.sample(logits, n, p);
}

// to_tile8 (kernels.cpp:971-991) of q4 pack rows, and row r of such a tiled matrix read back by the reference's own
// quad_row (kernels.cpp:1143)
__attribute__((visibility("default"))) void ref_to_tile8(int64_t rows, int64_t cols, const uint8_t *src, uint8_t *dst) {
    to_tile8(DType::Q4, rows, cols, src, dst);
}

__attribute__((visibility("default"))) void ref_tile8_row(const uint8_t *data, int64_t rows, int64_t cols, int64_t r,
                                                          uint8_t *out) {
    QView v = q4_view(data, rows, cols, 1.0f);
    v.quad = true;
    v.tile8 = true;
    quad_row(v, r, out);
}

}  // extern "C"
