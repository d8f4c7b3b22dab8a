// q4.hip - the q4 format on gfx950: the pack layout -> device layout permutation, dequantization, the RTN packer,
// int8 activation quantization (optionally fused with RMSNorm) and the dequant-in-register skinny GEMM.
//
// Reference arithmetic restated here (paths relative to the reference's engine/src):
//   dequant_row            kernels.cpp:1214-1228   level x (E4M3 x global), bit for bit
//   q4_block / e4m3_byte   yue2_q4.cpp:72-114       the packer's candidates and choice, bit for bit
//   quantize_activation    kernels.cpp:1254-1295   amax / 127 per 16 values, lrint, clamp +-127, bit for bit
//   rmsnorm                kernels.cpp:1520-1529   double sum of squares, 1 / sqrt(float(ss / n) + eps), x inv (1 + w)
//   matvec_rows_q_ref      kernels.cpp:1304-1322   integer block sums (exact), block scale e4m3 x act scale, fp32
//                                                  accumulation (here per k-lane then a fixed xor tree)
#include "common.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"

namespace gv {

// ---------------------------------------------------------------- layout
namespace {
// pack code c -> affine c' (level 2c' - 15): 0..7 (levels 1..15) -> 8..15, 8..15 (levels -1..-15) -> 7..0
__device__ inline uint32_t affine_nibbles(uint32_t w) {
    // per nibble: c < 8 ? c + 8 : 15 - c, i.e. c ^ 8 or c ^ 15, on all 8 nibbles at once
    const uint32_t neg = ((w & 0x88888888u) >> 3) * 0xFu;   // 0xF where c >= 8
    return w ^ (neg | 0x88888888u);
}
}  // namespace

__global__ void q4_from_pack_kernel(const uint8_t *__restrict__ pack, int64_t rows, int64_t cols, int S, int groups,
                                   uint8_t *__restrict__ codes, uint8_t *__restrict__ scales) {
    const int64_t nch = cols / 32;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * nch) return;
    const int64_t r = i / nch, c = i % nch;
    const size_t rb = static_cast<size_t>(cols / 16) * 9;
    const uint8_t *row = pack + static_cast<size_t>(r) * rb;
    const uint4 w = *reinterpret_cast<const uint4 *>(row + c * 16);
    uint4 o;
    o.x = affine_nibbles(w.x);
    o.y = affine_nibbles(w.y);
    o.z = affine_nibbles(w.z);
    o.w = affine_nibbles(w.w);
    *reinterpret_cast<uint4 *>(codes + q4_code_offset(rows, cols, S, r, c)) = o;
    uint8_t *sd = scales + q4_scale_offset(rows, S, groups, r, c);
    sd[0] = row[cols / 2 + 2 * c];
    sd[1] = row[cols / 2 + 2 * c + 1];
}

int q4_from_pack(const uint8_t *pack_dev, int64_t rows, int64_t cols, float global, uint8_t *codes, uint8_t *scales,
                 Q4 &out, hipStream_t st) {
    GV_REQUIRE(rows > 0 && cols > 0 && cols % 32 == 0, "q4: cols must be a positive multiple of 32");
    const int S = q4_lanes_for(cols);
    GV_REQUIRE(cols % (32 * S) == 0, "q4: cols must be a multiple of 32 x the k-lanes");
    const int steps = static_cast<int>(cols / (32 * S)), groups = q4_groups(steps);
    if (groups * 8 != steps) GV_CHECK_HIP(hipMemsetAsync(scales, 0, q4_scale_bytes(rows, cols), st));
    const int64_t n = rows * (cols / 32);
    hipLaunchKernelGGL(q4_from_pack_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, pack_dev,
                       rows, cols, S, groups, codes, scales);
    GV_CHECK_HIP(hipGetLastError());
    out.codes = codes;
    out.scales = scales;
    out.rows = rows;
    out.cols = cols;
    out.S = S;
    out.steps = steps;
    out.global = global;
    return 0;
}

// ---------------------------------------------------------------- dequant (kernels.cpp:1214-1228)
__global__ void q4_dequant_kernel(Q4 w, float *__restrict__ out) {
    const int64_t nch = w.cols / 32;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= w.rows * nch) return;
    const int64_t r = i / nch, c = i % nch;
    const uint4 cw = *reinterpret_cast<const uint4 *>(w.codes + q4_code_offset(w.rows, w.cols, w.S, r, c));
    const uint8_t *sd = w.scales + q4_scale_offset(w.rows, w.S, q4_groups(w.steps), r, c);
    const uint32_t words[4] = {cw.x, cw.y, cw.z, cw.w};
    float *o = out + r * w.cols + c * 32;
    for (int j = 0; j < 2; ++j) {
        const float s = __fmul_rn(e4m3_to_f32(sd[j]), w.global);   // E4M3 x global, then level x that
        for (int q = 0; q < 2; ++q) {
            const uint32_t wd = words[2 * j + q];
            for (int b = 0; b < 8; ++b) {
                const int cp = static_cast<int>((wd >> (4 * b)) & 15u);
                o[16 * j + 8 * q + b] = __fmul_rn(static_cast<float>(2 * cp - 15), s);
            }
        }
    }
}

int q4_dequant(const Q4 &w, float *out, hipStream_t st) {
    const int64_t n = w.rows * (w.cols / 32);
    hipLaunchKernelGGL(q4_dequant_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, w, out);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- the RTN packer (yue2_q4.cpp:72-114, :332-358)
__constant__ float c_e4m3_pos[127];   // E4M3's finite non-negative values, codes 0x00..0x7E

__device__ inline int e4m3_byte_dev(float x) {
    if (!(x > 0.0f)) return 0;
    if (x >= c_e4m3_pos[126]) return 126;
    int lo = 0, hi = 126;   // invariant: v[lo] <= x < v[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (c_e4m3_pos[mid] <= x) lo = mid;
        else hi = mid;
    }
    const float dl = __fsub_rn(x, c_e4m3_pos[lo]), dh = __fsub_rn(c_e4m3_pos[hi], x);
    if (dl < dh) return lo;
    if (dh < dl) return hi;
    return lo % 2 == 0 ? lo : hi;
}

__global__ void absmax_kernel(const float *__restrict__ w, int64_t n, unsigned int *__restrict__ out) {
    float m = 0.0f;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        m = fmaxf(m, fabsf(w[i]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));   // non-negative floats order as their bits
}

__global__ void q4_pack_kernel(const float *__restrict__ w, int64_t rows, int64_t cols,
                               const unsigned int *__restrict__ wmax_bits, uint8_t *__restrict__ out,
                               float *__restrict__ global_out) {
    const int64_t nb = cols / 16;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    // s2 = max|w| x 1.25 / (15 x 448)
    const float s2 = __fdiv_rn(__fmul_rn(__uint_as_float(*wmax_bits), 1.25f), 6720.0f);
    if (i == 0 && global_out) *global_out = s2;
    if (i >= rows * nb) return;
    const int64_t r = i / nb, blk = i % nb;
    const float *x = w + r * cols + blk * 16;
    float xv[16];
    float amax = 0.0f;
    for (int j = 0; j < 16; ++j) {
        xv[j] = x[j];
        amax = fmaxf(amax, fabsf(xv[j]));
    }
    int cand[10], nc = 0;
    const float ts[2] = {15.0f, 13.0f};
    for (int ti = 0; ti < 2; ++ti) {
        const int b0 = e4m3_byte_dev(__fdiv_rn(amax, __fmul_rn(ts[ti], s2)));
        for (int k = -2; k <= 2; ++k) cand[nc++] = min(max(b0 + k, 0), 0x7E);
    }
    float best = __builtin_inff();
    uint32_t best_codes[2] = {0, 0};
    int best_sb = 0;
    for (int c = 0; c < nc; ++c) {
        const float scale = __fmul_rn(c_e4m3_pos[cand[c]], s2), safe = scale == 0.0f ? 1.0f : scale;
        float err = 0.0f;
        uint32_t codes[2] = {0, 0};
        for (int j = 0; j < 16; ++j) {
            const float y = __fdiv_rn(xv[j], safe), a = fminf(fabsf(y), 15.0f);
            const int idx = min(max(static_cast<int>(rintf(__fmul_rn(__fsub_rn(a, 1.0f), 0.5f))), 0), 7);
            const bool neg = y < 0.0f;
            const float q = __fmul_rn(static_cast<float>(neg ? -(2 * idx + 1) : 2 * idx + 1), scale);
            const float d = __fsub_rn(q, xv[j]);
            err = __fadd_rn(err, __fmul_rn(d, d));
            codes[j / 8] |= static_cast<uint32_t>(idx + (neg ? 8 : 0)) << (4 * (j % 8));
        }
        if (err < best) {
            best = err;
            best_sb = cand[c];
            best_codes[0] = codes[0];
            best_codes[1] = codes[1];
        }
    }
    uint8_t *o = out + static_cast<size_t>(r) * (nb * 9);
    *reinterpret_cast<uint2 *>(o + blk * 8) = make_uint2(best_codes[0], best_codes[1]);
    o[nb * 8 + blk] = static_cast<uint8_t>(best_sb);
}

int q4_init_constants() {
    static bool done = false;
    if (done) return 0;
    float v[127];
    for (int b = 0; b < 127; ++b) {
        const int ex = (b >> 3) & 15, man = b & 7;
        v[b] = ex == 0 ? static_cast<float>(man) / 8.0f / 64.0f : (1.0f + static_cast<float>(man) / 8.0f) *
                                                                        static_cast<float>(1 << ex) / 128.0f;
    }
    GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(c_e4m3_pos), v, sizeof v));
    done = true;
    return 0;
}

int q4_pack(const float *w, int64_t rows, int64_t cols, unsigned int *scratch_u32, uint8_t *out, float *global_out,
            hipStream_t st) {
    GV_REQUIRE(cols % 16 == 0 && rows > 0, "q4_pack: cols must be a multiple of 16");
    if (q4_init_constants() != 0) return -1;
    GV_CHECK_HIP(hipMemsetAsync(scratch_u32, 0, 4, st));
    const int64_t n = rows * cols;
    hipLaunchKernelGGL(absmax_kernel, dim3(static_cast<unsigned>(std::min<int64_t>(4096, (n + 255) / 256))), dim3(256),
                       0, st, w, n, scratch_u32);
    const int64_t nb = rows * (cols / 16);
    hipLaunchKernelGGL(q4_pack_kernel, dim3(static_cast<unsigned>((nb + 255) / 256)), dim3(256), 0, st, w, rows, cols,
                       scratch_u32, out, global_out);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- activations
// One workgroup per token: optional RMSNorm (kernels.cpp:1520-1529), then the int8 blocks in the products' layout
// (common.hpp), and optionally the normalized fp32 row (the router's and the shared gate's input).
__global__ __launch_bounds__(256) void quantize_act_kernel(const float *__restrict__ x, int64_t ldx, int cols,
                                                           const float *__restrict__ norm_w, float eps,
                                                           uint8_t *__restrict__ act, int64_t act_stride,
                                                           float *__restrict__ h_out, int64_t ldh) {
    const int t = blockIdx.x;
    const float *xr = x + t * ldx;
    __shared__ double red[256];
    __shared__ float inv_s;
    float inv = 1.0f;
    if (norm_w) {
        double ss = 0.0;
        for (int i = threadIdx.x; i < cols; i += 256) ss += static_cast<double>(xr[i]) * static_cast<double>(xr[i]);
        red[threadIdx.x] = ss;
        __syncthreads();
        for (int o = 128; o > 0; o >>= 1) {
            if (static_cast<int>(threadIdx.x) < o) red[threadIdx.x] += red[threadIdx.x + o];
            __syncthreads();
        }
        if (threadIdx.x == 0)
            inv_s = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(red[0] / static_cast<double>(cols)), eps)));
        __syncthreads();
        inv = inv_s;
    }
    uint8_t *ar = act + t * act_stride;
    for (int b = threadIdx.x; b < cols / 16; b += 256) {
        float v[16];
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const int c = b * 16 + i;
            float y = xr[c];
            if (norm_w) y = __fmul_rn(__fmul_rn(y, inv), __fadd_rn(1.0f, norm_w[c]));
            v[i] = y;
            amax = fmaxf(amax, fabsf(y));
        }
        if (h_out)
            for (int i = 0; i < 16; ++i) h_out[t * ldh + b * 16 + i] = v[i];
        const float s = __fdiv_rn(amax, 127.0f), qi = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        int sum = 0;
        uint32_t dw[4] = {0, 0, 0, 0};   // word 0: even, odd; word 1: even, odd
        for (int i = 0; i < 16; ++i) {
            const int q = min(max(static_cast<int>(rintf(__fmul_rn(v[i], qi))), -127), 127);
            sum += q;
            const int word = i / 8, within = i % 8;
            dw[2 * word + (within & 1)] |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * (within >> 1));
        }
        const int c = b / 2, j = b % 2;
        uint8_t *chunk = ar + static_cast<size_t>(c) * kActChunkBytes;
        *reinterpret_cast<uint4 *>(chunk + 16 * j) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
        reinterpret_cast<float *>(chunk + 32)[j] = s;
        reinterpret_cast<int *>(chunk + 40)[j] = -15 * sum;
    }
}

int quantize_act(const float *x, int64_t ldx, int M, int cols, const float *norm_w, float eps, uint8_t *act,
                 int64_t act_stride, float *h_out, int64_t ldh, hipStream_t st) {
    GV_REQUIRE(cols % 32 == 0 && M > 0, "quantize_act: cols must be a multiple of 32");
    hipLaunchKernelGGL(quantize_act_kernel, dim3(M), dim3(256), 0, st, x, ldx, cols, norm_w, eps, act, act_stride,
                       h_out, ldh);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- the skinny GEMM (gemv_core.hpp)
template <int S, int R, int MT>
__global__ __launch_bounds__(256) void gemv_q4_kernel(Q4 w, const uint8_t *__restrict__ act, int64_t act_stride,
                                                      int M, GemvOut out) {
    constexpr int G = 64 / S;
    constexpr int WROWS = G * R;
    extern __shared__ uint4 lds_u4[];
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds_u4);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane / S, k = lane % S;
    const int64_t abytes = (w.cols / 32) * kActChunkBytes;
    load_acts(lds, act, act_stride, abytes, M);
    __syncthreads();
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * WROWS;
    if (row0 >= w.rows) return;
    float acc[R][MT];
    gemv_wave<S, R, MT>(w.codes, w.scales, w.rows, w.cols, w.steps, row0, lds, abytes, M, g, k, acc);
    gemv_reduce<S, R, MT>(acc, M);
    if (k != 0) return;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int64_t row = row0 + i * G + g;
        if (row >= w.rows) continue;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= M) break;
            out.put(row, t, acc[i][t]);
        }
    }
}

template <int S, int R, int MT>
static int launch_gemv(const Q4 &w, const uint8_t *act, int64_t act_stride, int M, const GemvOut &out,
                       hipStream_t st) {
    constexpr int WROWS = (64 / S) * R;
    const int64_t wg = (w.rows + 4 * WROWS - 1) / (4 * WROWS);
    const size_t lds = static_cast<size_t>(M) * act_bytes(w.cols);
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_kernel<S, R, MT>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL((gemv_q4_kernel<S, R, MT>), dim3(static_cast<unsigned>(wg)), dim3(256), lds, st, w, act,
                       act_stride, M, out);
    return 0;
}

template <int S, int R>
static int dispatch_mt(const Q4 &w, const uint8_t *act, int64_t act_stride, int M, const GemvOut &out,
                       hipStream_t st) {
    if (M <= 1) return launch_gemv<S, R, 1>(w, act, act_stride, M, out, st);
    if (M <= 2) return launch_gemv<S, R, 2>(w, act, act_stride, M, out, st);
    if (M <= 4) return launch_gemv<S, R, 4>(w, act, act_stride, M, out, st);
    if (M <= 8) return launch_gemv<S, R, 8>(w, act, act_stride, M, out, st);
    if (M <= 16) return launch_gemv<S, (R > 2 ? 2 : R), 16>(w, act, act_stride, M, out, st);
    return launch_gemv<S, 1, 32>(w, act, act_stride, M, out, st);
}

int gemv_q4(const Q4 &w, const uint8_t *act, int64_t act_stride, int M, const GemvOut &out, hipStream_t st) {
    GV_REQUIRE(M >= 1 && M <= kMaxRows, "gemv_q4: 1 <= M <= 32 tokens");
    GV_REQUIRE(static_cast<size_t>(M) * act_bytes(w.cols) <= 160 * 1024, "gemv_q4: activations exceed LDS");
    // rows a lane: as many as keep >= 512 workgroups (a large matrix takes 4, a small one 1)
    const int64_t G = 64 / w.S;
    const int R = w.rows >= 512 * 4 * G * 4 ? 4 : w.rows >= 512 * 4 * G * 2 ? 2 : 1;
    int rc;
    switch (w.S * 8 + R) {
    case 1 * 8 + 1: case 1 * 8 + 2: case 1 * 8 + 4: rc = dispatch_mt<1, 1>(w, act, act_stride, M, out, st); break;
    case 2 * 8 + 1: rc = dispatch_mt<2, 1>(w, act, act_stride, M, out, st); break;
    case 2 * 8 + 2: case 2 * 8 + 4: rc = dispatch_mt<2, 2>(w, act, act_stride, M, out, st); break;
    case 4 * 8 + 1: rc = dispatch_mt<4, 1>(w, act, act_stride, M, out, st); break;
    case 4 * 8 + 2: case 4 * 8 + 4: rc = dispatch_mt<4, 2>(w, act, act_stride, M, out, st); break;
    case 8 * 8 + 1: rc = dispatch_mt<8, 1>(w, act, act_stride, M, out, st); break;
    case 8 * 8 + 2: rc = dispatch_mt<8, 2>(w, act, act_stride, M, out, st); break;
    case 8 * 8 + 4: rc = dispatch_mt<8, 4>(w, act, act_stride, M, out, st); break;
    default: set_error("gemv_q4: unsupported k-lane count"); return -1;
    }
    if (rc != 0) return rc;
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace gv
