// common.hpp - device helpers shared by the gfx950 kernels of libgeode_verify.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace gv {

// ---------------------------------------------------------------- errors
// The last error of the calling thread (gv_last_error); every entry point returns nonzero and sets it on failure.
void set_error(const std::string &msg);
const char *last_error();

#define GV_CHECK_HIP(expr)                                                                          \
    do {                                                                                            \
        hipError_t e_ = (expr);                                                                     \
        if (e_ != hipSuccess) {                                                                     \
            ::gv::set_error(std::string(#expr) + ": " + hipGetErrorString(e_));                     \
            return -1;                                                                              \
        }                                                                                           \
    } while (0)

#define GV_REQUIRE(cond, msg)                                                                       \
    do {                                                                                            \
        if (!(cond)) {                                                                              \
            ::gv::set_error(msg);                                                                   \
            return -1;                                                                              \
        }                                                                                           \
    } while (0)

// Dynamic LDS above 64 KB must be granted per kernel; asks for `bytes` when the kernel's grant is smaller.
inline int lds_grant(const void *kernel, size_t bytes, int &granted) {
    if (bytes <= 64 * 1024 || static_cast<int>(bytes) <= granted) return 0;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(std::string("LDS of ") + std::to_string(bytes) + " bytes refused: " + hipGetErrorString(e));
        return -1;
    }
    granted = static_cast<int>(bytes);
    return 0;
}

// ---------------------------------------------------------------- a q4 matrix on the device
// (the tile layout of mfma_gemv.hpp; global applied to the products' sums)
struct Q4 {
    const uint8_t *codes = nullptr;
    const uint8_t *scales = nullptr;
    int64_t rows = 0, cols = 0;
    int S = 0, steps = 0;   // (unused by the tile layout; kept for the C ABI's struct)
    float global = 1.0f;
};

inline int64_t q4_tile_rows(int64_t rows) { return (rows + 15) / 16 * 16; }
inline size_t q4_code_bytes(int64_t rows, int64_t cols) { return static_cast<size_t>(q4_tile_rows(rows)) * static_cast<size_t>(cols / 2); }
inline size_t q4_scale_bytes(int64_t rows, int64_t cols) { return static_cast<size_t>(q4_tile_rows(rows)) * static_cast<size_t>(cols / 16); }
// one row's activations for the products: cols fp16 hi + lo halves (mfma_gemv.hpp)
inline size_t act_bytes(int64_t cols) { return static_cast<size_t>(cols) * 4; }
__host__ __device__ inline int64_t act_halves(int64_t cols) { return cols * 2; }

// ---------------------------------------------------------------- device helpers
__device__ inline float e4m3_to_f32(uint32_t b) {
    // E4M3FN as half bits: exponent and mantissa moved into place, then 2^8 for the bias (15 - 7); exact for every
    // finite byte (0x7F / 0xFF, the NaNs, are never written by the packer)
    const uint16_t hb = static_cast<uint16_t>(((b & 0x80u) << 8) | ((b & 0x7Fu) << 7));
    const _Float16 h = __builtin_bit_cast(_Float16, hb);
    return static_cast<float>(h) * 256.0f;
}

template <typename T>
__device__ inline T wave_sum_xor(T v, int width) {
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ inline float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace gv
