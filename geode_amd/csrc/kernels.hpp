// kernels.hpp - host-side launchers of the gfx950 kernels (namespace gv); the C ABI (capi.hip) sits on these.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace gv {

constexpr int kMaxRows = 32;   // rows (tokens) a skinny product takes at once

// Where a product's results go: y[t * ldy + row] = acc x global (the global of the row's segment: a fused matrix
// of parts, e.g. q | k | v, keeps each part's own), or += when accumulate (the residual add).
struct GemvOut {
    float *y = nullptr;
    int64_t ldy = 0;
    int accumulate = 0;
    int nseg = 1;
    int64_t seg_end[4] = {0, 0, 0, 0};
    float seg_global[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    int trace_cls = -1;   // the kernel class whose clock stamps the launch writes (a measurement aid; -1: none)
    __device__ inline float scaled(int64_t row, float v) const {   // v x the row's global
        float g = seg_global[0];
        for (int s = 1; s < nseg; ++s)
            if (row >= seg_end[s - 1]) g = seg_global[s];
        return v * g;
    }
    __device__ inline void put(int64_t row, int t, float v) const {
        const float r = scaled(row, v);
        float *p = y + t * ldy + row;
        if (accumulate) *p += r;
        else *p = r;
    }
};

inline GemvOut gemv_out(float *y, int64_t ldy, float global, int accumulate = 0) {
    GemvOut o;
    o.y = y;
    o.ldy = ldy;
    o.accumulate = accumulate;
    o.nseg = 1;
    o.seg_end[0] = INT64_MAX;
    o.seg_global[0] = global;
    return o;
}

int q4_init_constants();
int q4_from_pack(const uint8_t *pack_dev, int64_t rows, int64_t cols, float global, uint8_t *codes, uint8_t *scales,
                 Q4 &out, hipStream_t st);
int q4_dequant(const Q4 &w, float *out, hipStream_t st);
int q4_pack(const float *w, int64_t rows, int64_t cols, unsigned int *scratch_u32, uint8_t *out, float *global_out,
            hipStream_t st);
// act rows: act_bytes(cols) apart (act_stride in halves), the int8 path's values
int quantize_act(const float *x, int64_t ldx, int M, int cols, const float *norm_w, float eps, _Float16 *act,
                 int64_t act_stride, float *h_out, int64_t ldh, hipStream_t st);
int trace_set_q4(uint64_t *p);   // the gemv kernels' g_trace (q4.hip)
int trace_set_gdn(uint64_t *p);  // the Gated DeltaNet kernel's g_trace (gdn.hip)
// the products' operands of every source file's kernels: the int8 path's (0) or the exact path's (1) (mfma_gemv.hpp
// g_act_exact); use_act_mode switches them all when the mode differs from the current one, waiting for the device
int act_mode_set_model(int exact);
int act_mode_set_q4(int exact);
int act_mode_set_gdn(int exact);
int act_mode_set_mtp(int exact);
int act_mode_set_prefill(int exact);
int use_act_mode(int exact);
int gemv_q4(const Q4 &w, const _Float16 *act, int64_t act_stride, int M, const GemvOut &out, hipStream_t st);
// C1's dense FFN pieces: fp16 rows to operands; gate and up with the SwiGLU and its quantization (M <= 8)
int quantize_f16(const uint16_t *x, int M, int cols, _Float16 *act, int64_t act_stride, hipStream_t st);
int ffn_up(const Q4 &gate, const Q4 &up, const _Float16 *act, int64_t act_stride, int M, _Float16 *act_m,
           int64_t act_m_stride, hipStream_t st);
// the waves a product's K (a multiple of 128) splits over and the 32-value chunks each takes, for ntt 16-row tiles
// of activations; 0 when one launch cannot take K (more than 8 waves)
int mfma_split(int64_t K, int ntt, int &waves, int &kw);
int64_t tiles_per_wg(int64_t ntiles, int waves, int ntt);

// the library's stream and lazy device set-up (capi.hip)
hipStream_t stream();
int ensure_init();

// elementwise helpers (misc.hip)
int f16_to_f32(const uint16_t *x, int64_t n, float *y, hipStream_t st);
int copy16(const void *src, int64_t n16, void *dst, hipStream_t st);   // n16 16-byte words, both 16-byte aligned
int swiglu(const float *g, const float *u, int64_t n, float *m, hipStream_t st);
int fill_normal(uint64_t seed, int64_t n, float sigma, float *out, hipStream_t st);

}  // namespace gv
