// oracle_internal.hpp - helpers shared by the oracle's translation units (test infrastructure only).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <vector>

namespace orc {

struct QAct {   // kernels.hpp:96-107 (natural order only: the lane orders are NEON's)
    std::vector<int8_t> q;
    std::vector<float> scale;
    std::vector<int32_t> bsum;
};

uint64_t splitmix64(uint64_t x);
uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);
uint16_t f32_to_bf16(float f);
inline float bf16_to_f32(uint16_t v) {
    const uint32_t u = static_cast<uint32_t>(v) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

void par(int64_t items, int64_t chunk, const std::function<void(int64_t, int64_t)> &fn);

const float *e4m3_table();
void matvec_exact(const uint8_t *w, int64_t cols, float global, const float *x, float *y, int64_t r0, int64_t r1);
void quantize(const float *x, int64_t cols, QAct &a);
void matvec_q(const uint8_t *w, int64_t cols, float global, const QAct &a, float *y, int64_t r0, int64_t r1);
void bf16_rows(const uint16_t *w, int64_t cols, int n, const float *const *xs, float *const *ys, int64_t r0, int64_t r1);
void rmsnorm(const float *x, const float *w, float *out, int n, float eps, bool zero_centered);
void route_topk(const float *logits, int E, int K, int *ids, float *weights);
void matmul(const uint8_t *w, int64_t rows, int64_t cols, float global, int n, const float *const *xs,
            float *const *ys, int mode);

inline size_t q4_row_bytes(int64_t cols) { return static_cast<size_t>(cols / 16) * 9; }
inline float silu(float x) { return x / (1.0f + std::exp(-x)); }   // kernels.hpp:141
inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

}  // namespace orc
