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
// the scales: per 16-row tile, per quad of four 128-value super-chunks, 512 bytes (a lane's four words adjacent)
inline size_t q4_scale_bytes(int64_t rows, int64_t cols) {
    return static_cast<size_t>(q4_tile_rows(rows) / 16) * static_cast<size_t>((cols / 128 + 3) / 4) * 512;
}
// one row's activations for the products: cols fp16 hi + lo halves (mfma_gemv.hpp)
inline size_t act_bytes(int64_t cols) { return static_cast<size_t>(cols) * 4; }
__host__ __device__ inline int64_t act_halves(int64_t cols) { return cols * 2; }

// ---------------------------------------------------------------- data exchanged within one launch
// Workgroups of one launch on different XCDs do not share an L2: a plain store may sit in the writer's L2 and a plain
// load may hit a stale line in the reader's. Buffer loads and stores with the sc1 cache policy (gfx940+: device
// scope) are coherent across the XCDs without a cache maintenance operation (no L2 write-back or invalidate, which on
// gfx950 costs about as much as a kernel boundary). Every buffer one workgroup writes and another reads later in the
// same launch goes through these; a producer then waits for its stores and bumps a counter (relaxed, device scope),
// and its consumers poll the counter before loading. `base` must be uniform across the wave; offsets in bytes.
typedef uint32_t xu4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;   // the sc1 bit of the buffer instructions' cache policy operand
__device__ inline __amdgpu_buffer_rsrc_t xrs(const void *base) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32));
    void *p = reinterpret_cast<void *>((static_cast<uint64_t>(hi) << 32) | lo);
    // (num_records: the whole 31-bit range; word 3: the 32-bit data format gfx9 buffer accesses require)
    return __builtin_amdgcn_make_buffer_rsrc(p, static_cast<short>(0), 0x7FFFFFFF, 0x00020000);
}
__device__ inline xu4 xld16(const void *base, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(xrs(base), off, 0, kSc1);
}
__device__ inline void xst16(void *base, uint32_t off, xu4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, xrs(base), off, 0, kSc1); }
__device__ inline float xldf(const float *base, uint32_t i) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs(base), i * 4u, 0, kSc1));
}
__device__ inline void xstf(float *base, uint32_t i, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), xrs(base), i * 4u, 0, kSc1);
}
__device__ inline float4 xld4f(const float *base, uint32_t i) { return __builtin_bit_cast(float4, xld16(base, i * 4u)); }
__device__ inline void xst4f(float *base, uint32_t i, float4 v) { xst16(base, i * 4u, __builtin_bit_cast(xu4, v)); }

// The producer side: every thread's stores complete, then the workgroup's own flag word is set (a device-scope store;
// one word a producer: many workgroups bumping one counter serialize at the memory side, ~40 ns each).
__device__ inline void signal_done(int *flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's stores acknowledged (gfx9: vmcnt counts them)
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The consumer side: the first wave polls the n producers' flags (device-scope loads, a few per lane) until every one
// is set, then the workgroup goes on. Producers always have lower workgroup ids than their consumers (workgroups are
// dispatched in id order), so they are resident or done and never wait themselves: the wait ends. A bound on the
// polls all the same (~0.1 s): past it the flag err is set (the host reports it) and the workgroup goes on, so no wave
// can spin forever.
constexpr int kMaxPolls = 1 << 17;
__device__ inline void wait_flags(const int *flags, int n, int *err) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        for (int polls = 0;; ++polls) {
            int ok = 1;
            for (int i = lane; i < n; i += 64) ok &= __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
            if (__all(ok)) break;
            if (polls > kMaxPolls) {
                if (lane == 0) __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}
// Every flag of [0, n) back to zero for the launch's next use (by the launch's last consumer, once every other
// workgroup has passed its waits)
__device__ inline void clear_flags(int *flags, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) __hip_atomic_store(flags + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- a measurement aid: workgroup clock stamps
// When a translation unit's g_trace is set (gv_model_trace; each source file's kernels have their own copy), thread 0
// of each workgroup of the traced kernels writes the 100 MHz clock (s_memrealtime) at a few points to
// g_trace[(cls * kTraceWgs + workgroup) * 8 + slot]; each launch overwrites its class's stamps, so after a step they
// are the last layer's. Null (the default): a scalar load (constant memory, cached) and a branch a stamp.
constexpr int kTraceWgs = 8192;
static __constant__ uint64_t *g_trace;
__device__ inline void trace(int cls, int slot) {
    uint64_t *t = g_trace;
    if (t && threadIdx.x == 0 && blockIdx.x < kTraceWgs) {
        uint64_t *w = t + (static_cast<size_t>(cls) * kTraceWgs + blockIdx.x) * 8;
        w[slot] = __builtin_amdgcn_s_memrealtime();
        if (slot == 0)   // where the workgroup runs: XCC id (high word) and HW_ID (CU, SH, SE: low word)
            w[7] = (static_cast<uint64_t>(__builtin_amdgcn_s_getreg(0xF814)) << 32) | __builtin_amdgcn_s_getreg(0xF804);
    }
}

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

// y as two fp16 halves, hi = y rounded to fp16 and lo = (y - hi) rounded, so hi + lo = y to 2^-22 relative. The
// empty asm pins y as a computed fp32 value: without it the compiler may fold the product that made y into the
// conversion (one rounding, v_fma_mix) for one use of hi and not for another, and hi + lo is then off by an ulp.
__device__ inline void split_f16(float y, _Float16 &hi, _Float16 &lo) {
    asm volatile("" : "+v"(y));
    hi = static_cast<_Float16>(y);
    lo = static_cast<_Float16>(y - static_cast<float>(hi));
}

// y rounded to fp16 from its fp32 value: when y is a product, two roundings (fp32, then fp16), as the reference's
// fp32 result stored to an fp16 cache. The empty asm keeps the compiler from folding the product into the
// conversion (v_fma_mixlo_f16, one rounding), which it does in some kernels and not in others.
__device__ inline _Float16 f16_of(float y) {
    asm volatile("" : "+v"(y));
    return static_cast<_Float16>(y);
}

// DPP lane moves within 16-lane rows (quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror = 0x141,
// row_mirror = 0x140): full-rate VALU, no LDS crossbar round trip
template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ inline double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u)), CTRL, 0xF, 0xF, false);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(u >> 32)), CTRL, 0xF, 0xF,
                                                    false);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// the value of lane l ^ 8 (the other half of the lane's 16-lane row): DPP row_ror:8, no LDS crossbar round trip
__device__ inline float xor8(float v) { return dpp_f<0x128>(v); }

// The wave reductions, in vector registers throughout (no LDS crossbar round trip): pairs, quads, 8s and 16s of lanes
// within each 16-lane row by DPP (every lane then holds its row's value), then the rows by DPP row broadcasts (gfx9:
// row 1 += row 0's lane 15 and row 3 += row 2's, then row 3 += row 1's lane 31), and lane 63's value read out as a
// uniform one: the sum (row 0 + row 1) + (row 2 + row 3), the same bits whatever the lanes' order within a row pair
template <int CTRL, int ROWS = 0xF>
__device__ inline uint32_t dpp_u(uint32_t old, uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL, ROWS, 0xF, false));
}
template <int CTRL, int ROWS = 0xF>
__device__ inline double dpp_dd(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp_u<CTRL, ROWS>(0u, static_cast<uint32_t>(u));
    const uint32_t hi = dpp_u<CTRL, ROWS>(0u, static_cast<uint32_t>(u >> 32));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ inline float lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ inline double wave_sum(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    v += dpp_dd<0x142, 0xA>(v);   // rows 1, 3: + lane 15 of rows 0, 2 (rows 0, 2: + 0)
    v += dpp_dd<0x143, 0xC>(v);   // rows 2, 3: + lane 31
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u)), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(u >> 32)), 63));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ inline float wave_sum_f(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    v += __builtin_bit_cast(float, dpp_u<0x142, 0xA>(0u, __builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp_u<0x143, 0xC>(0u, __builtin_bit_cast(uint32_t, v)));
    return lane63(v);
}

// the inclusive prefix sum over the wave's lanes (integers, exact): shifts 1, 2, 4, 8 within each 16-lane row, then
// the rows' totals carried by row broadcasts
__device__ inline int wave_incl_scan(int v) {
    v += static_cast<int>(dpp_u<0x111>(0u, static_cast<uint32_t>(v)));   // row_shr:1 (lane 0 of a row: + 0)
    v += static_cast<int>(dpp_u<0x112>(0u, static_cast<uint32_t>(v)));   // row_shr:2
    v += static_cast<int>(dpp_u<0x114>(0u, static_cast<uint32_t>(v)));   // row_shr:4
    v += static_cast<int>(dpp_u<0x118>(0u, static_cast<uint32_t>(v)));   // row_shr:8
    v += static_cast<int>(dpp_u<0x142, 0xA>(0u, static_cast<uint32_t>(v)));   // rows 1, 3: + lane 15 of rows 0, 2
    v += static_cast<int>(dpp_u<0x143, 0xC>(0u, static_cast<uint32_t>(v)));   // rows 2, 3: + lane 31
    return v;
}

// The wave's largest of int keys, in every lane: four DPP steps within each 16-lane row (pairs, quads, eights,
// sixteens), then gfx950's row swaps (rows 0 <-> 1 and 2 <-> 3, then the halves), no lane read back. For non-negative
// floats the keys are their bits (the order is the same).
__device__ inline int wave_max_all_i(int v) {
    // (every lane's source is a lane of its own row: no bound is hit; each step becomes one v_max_i32_dpp)
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true));    // quad_perm [1, 0, 3, 2]
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true));    // quad_perm [2, 3, 0, 1]
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true));   // row_half_mirror
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true));   // row_mirror
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);      // {rows 0 0 2 2, rows 1 1 3 3}
    v = max(static_cast<int>(r[0]), static_cast<int>(r[1]));
    const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);      // {low half twice, high half twice}
    return max(static_cast<int>(h[0]), static_cast<int>(h[1]));
}

// the largest float over the wave's 64 lanes, in every lane (signed floats as order-preserving int keys: a negative
// value's magnitude bits flipped)
__device__ inline float wave_max_all_f(float v) {
    const int b = __float_as_int(v);
    const int k = wave_max_all_i(b < 0 ? b ^ 0x7FFFFFFF : b);
    return __int_as_float(k < 0 ? k ^ 0x7FFFFFFF : k);
}

// the maximum over the wave's 64 lanes, a uniform value
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    v = fmaxf(v, __builtin_bit_cast(float, dpp_u<0x142, 0xA>(u, u)));   // rows 0, 2 keep their own value
    const uint32_t u2 = __builtin_bit_cast(uint32_t, v);
    v = fmaxf(v, __builtin_bit_cast(float, dpp_u<0x143, 0xC>(u2, u2)));
    return lane63(v);
}

}  // namespace gv
