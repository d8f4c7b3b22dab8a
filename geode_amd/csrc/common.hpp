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

// ---------------------------------------------------------------- the device q4 layout
// A q4 matrix as the kernels read it (the pack's bytes permuted, nothing lost; gv_q4_from_pack makes it):
//  * codes: the pack's nibbles in the affine order c' (level = 2c' - 15: pack code c < 8 -> c + 8, c >= 8 ->
//    15 - c), value 2j in the low nibble of byte j of a 32-value chunk as in the pack;
//  * a row's 32-value chunks c = s * S + k go to k-lane k (0..S-1) at step s (0..steps-1); rows in tiles of
//    kTileRows; inside a tile the 16-byte chunks are ordered [step][row][k-lane], so the lanes of one wave that
//    load step s of 64/S consecutive rows read 1 KB of consecutive bytes;
//  * scales: per (row, k-lane) the E4M3 bytes of its blocks, 8 steps (16 bytes) a group, ordered [group][row][k]
//    inside a tile: one 16-byte load gives a lane its scales for 8 steps.
constexpr int kTileRows = 256;

struct Q4 {
    const uint8_t *codes = nullptr;
    const uint8_t *scales = nullptr;
    int64_t rows = 0, cols = 0;
    int S = 1, steps = 0;
    float global = 1.0f;
};

inline int q4_lanes_for(int64_t cols) {   // k-lanes per row: 256+ columns each, at most 8
    int S = 1;
    while (S < 8 && cols >= 256 * 2 * S) S *= 2;
    return S;
}
__host__ __device__ inline int q4_groups(int steps) { return (steps + 7) / 8; }
inline size_t q4_code_bytes(int64_t rows, int64_t cols) { return static_cast<size_t>(rows) * static_cast<size_t>(cols / 2); }
inline size_t q4_scale_bytes(int64_t rows, int64_t cols) {
    const int S = q4_lanes_for(cols);
    const int steps = static_cast<int>(cols / (32 * S));
    return static_cast<size_t>(rows) * S * q4_groups(steps) * 16;
}

__host__ __device__ inline size_t q4_code_offset(int64_t rows, int64_t cols, int S, int64_t r, int64_t c) {
    const int64_t t = r / kTileRows, rho = r % kTileRows;
    const int64_t th = (rows - t * kTileRows) < kTileRows ? rows - t * kTileRows : kTileRows;
    const int64_t s = c / S, k = c % S;
    return static_cast<size_t>(t * kTileRows * (cols / 2) + ((s * th + rho) * S + k) * 16);
}
__host__ __device__ inline size_t q4_scale_offset(int64_t rows, int S, int groups, int64_t r, int64_t c) {
    const int64_t t = r / kTileRows, rho = r % kTileRows;
    const int64_t th = (rows - t * kTileRows) < kTileRows ? rows - t * kTileRows : kTileRows;
    const int64_t s = c / S, k = c % S;
    return static_cast<size_t>(t * kTileRows * S * groups * 16 + (((s / 8) * th + rho) * S + k) * 16 + (s % 8) * 2);
}

// ---------------------------------------------------------------- activations
// The int8 activations of one token as the products read them (quantize_activation's values, kernels.cpp:1254-1295):
// per 32-value chunk 48 bytes: the 32 int8 values as 8 dwords [even | odd] per 8-value word (the even values
// 0 2 4 6 then the odd ones 1 3 5 7: the order the code nibbles come out in), then the two blocks' scales
// (amax / 127) and their corrections -15 * (sum of the block's int8 values) for the affine codes.
constexpr int kActChunkBytes = 48;
inline size_t act_bytes(int64_t cols) { return static_cast<size_t>(cols / 32) * kActChunkBytes; }

// ---------------------------------------------------------------- device helpers
__device__ inline float e4m3_to_f32(uint32_t b) {
    // E4M3FN as half bits: exponent and mantissa moved into place, then 2^8 for the bias (15 - 7); exact for every
    // finite byte (0x7F / 0xFF, the NaNs, are never written by the packer)
    const uint16_t hb = static_cast<uint16_t>(((b & 0x80u) << 8) | ((b & 0x7Fu) << 7));
    const _Float16 h = __builtin_bit_cast(_Float16, hb);
    return static_cast<float>(h) * 256.0f;
}

__device__ inline int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
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
