// misc.hip - small elementwise kernels: fp16 widening, the seeded normal generator used for device-side synthetic
// weights, and the run-time error state.
#include <algorithm>
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace gv {

namespace {
thread_local std::string g_error;
}
void set_error(const std::string &msg) { g_error = msg; }
const char *last_error() { return g_error.c_str(); }

__global__ void f16_to_f32_kernel(const uint16_t *__restrict__ x, int64_t n, float *__restrict__ y) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = static_cast<float>(__builtin_bit_cast(_Float16, x[i]));
}

int f16_to_f32(const uint16_t *x, int64_t n, float *y, hipStream_t st) {
    hipLaunchKernelGGL(f16_to_f32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, x, n, y);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// a plain 16-byte vector copy (device to device); its known traffic also scales the HBM byte counters
__global__ void copy16_kernel(const uint4 *__restrict__ src, int64_t n, uint4 *__restrict__ dst) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

int copy16(const void *src, int64_t n16, void *dst, hipStream_t st) {
    const int64_t blocks = std::min<int64_t>((n16 + 255) / 256, 256 * 16);
    hipLaunchKernelGGL(copy16_kernel, dim3(static_cast<unsigned>(std::max<int64_t>(blocks, 1))), dim3(256), 0, st,
                       static_cast<const uint4 *>(src), n16, static_cast<uint4 *>(dst));
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// silu(g) * u (kernels.hpp:141: x / (1 + e^-x))
__global__ void swiglu_kernel(const float *__restrict__ g, const float *__restrict__ u, int64_t n,
                              float *__restrict__ m) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        m[i] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), u[i]);
    }
}

int swiglu(const float *g, const float *u, int64_t n, float *m, hipStream_t st) {
    hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, g, u, n, m);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// The oracle's generator (splitmix64 over seed x 0xD1342543DE82EF95 + i, Box-Muller in double): the same integer
// stream on every device, the transcendental functions the device's own.
__device__ inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    uint64_t z = x;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(uint64_t seed, int64_t n, float sigma, float *__restrict__ out) {
    const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;   // one Box-Muller pair
    if (2 * k >= n) return;
    const uint64_t base = seed * 0xD1342543DE82EF95ull;
    const double u1 = (static_cast<double>(splitmix64(base + 2 * static_cast<uint64_t>(k)) >> 11) + 0.5) * 0x1p-53;
    const double u2 = static_cast<double>(splitmix64(base + 2 * static_cast<uint64_t>(k) + 1) >> 11) * 0x1p-53;
    const double r = sqrt(-2.0 * log(u1));
    double s, c;
    sincospi(2.0 * u2, &s, &c);
    out[2 * k] = static_cast<float>(static_cast<double>(sigma) * r * c);
    if (2 * k + 1 < n) out[2 * k + 1] = static_cast<float>(static_cast<double>(sigma) * r * s);
}

int fill_normal(uint64_t seed, int64_t n, float sigma, float *out, hipStream_t st) {
    const int64_t pairs = (n + 1) / 2;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256), 0, st, seed, n,
                       sigma, out);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace gv
