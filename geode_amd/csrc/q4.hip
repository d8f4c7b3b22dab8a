// q4.hip - the q4 format on gfx950: the pack layout -> device layout permutation, dequantization, the RTN packer,
// int8 activation quantization (optionally fused with RMSNorm) and the dequant-in-register skinny GEMM.
//
// Reference arithmetic restated here (paths relative to the reference's engine/src):
//   dequant_row            kernels.cpp:1214-1228   level x (E4M3 x global), bit for bit
//   q4_block / e4m3_byte   yue2_q4.cpp:72-114       the packer's candidates and choice, bit for bit
//   quantize_activation    kernels.cpp:1254-1295   amax / 127 per 16 values, lrint, clamp +-127, bit for bit
//   rmsnorm                kernels.cpp:1520-1529   double sum of squares, 1 / sqrt(float(ss / n) + eps), x inv (1 + w)
//   matvec_rows_q_ref      kernels.cpp:1304-1322   the int8 path's products: exact weights x (q x act scale) on the
//                                                  matrix cores, fp32 sums (mfma_gemv.hpp)
#include "common.hpp"
#include "kernels.hpp"
#include "mfma_gemv.hpp"

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

// one thread per (row, 8-value code word): the pack's word w of row r into the tile layout (mfma_gemv.hpp)
__global__ void q4_from_pack_kernel(const uint8_t *__restrict__ pack, int64_t rows, int64_t cols,
                                    uint8_t *__restrict__ codes, uint8_t *__restrict__ scales) {
    const int64_t nw = cols / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * nw) return;
    const int64_t r = i / nw, wi = i % nw;
    const size_t rb = static_cast<size_t>(cols / 16) * 9;
    const uint8_t *row = pack + static_cast<size_t>(r) * rb;
    const uint32_t w = *reinterpret_cast<const uint32_t *>(row + wi * 4);
    const int64_t T = r / kTileR, rr = r % kTileR, nsc = cols / kSuperK;
    const int64_t sc = wi / 16, j = (wi % 16) / 4, g = wi % 4;   // word 16 sc + 4 j + g
    const int64_t blk = T * nsc + sc;
    *reinterpret_cast<uint32_t *>(codes + blk * 1024 + (rr + 16 * g) * 16 + j * 4) = tile_word(affine_nibbles(w));
    if (g % 2 == 0)   // the block of (chunk j, k-groups g, g + 1): pack scale 8 sc + 2 j + g / 2
        scales[tq4_scale_off(T, (nsc + 3) / 4, sc, rr, g, j)] = row[cols / 2 + 8 * sc + 2 * j + g / 2];
}

int q4_from_pack(const uint8_t *pack_dev, int64_t rows, int64_t cols, float global, uint8_t *codes, uint8_t *scales,
                 Q4 &out, hipStream_t st) {
    GV_REQUIRE(rows > 0 && cols > 0 && cols % kSuperK == 0, "q4: cols must be a positive multiple of 128");
    const int64_t nsc = cols / kSuperK, nsq = (nsc + 3) / 4;
    if (rows % kTileR != 0) {   // the last tile's missing rows: zero codes and scales (their sums are discarded)
        const int64_t T = rows / kTileR;
        GV_CHECK_HIP(hipMemsetAsync(codes + T * nsc * 1024, 0, nsc * 1024, st));
        GV_CHECK_HIP(hipMemsetAsync(scales + T * nsq * 512, 0, nsq * 512, st));
    }
    if (nsc % 4 != 0)   // the last quad's unused super-chunks: zero scales (never read, kept defined)
        GV_CHECK_HIP(hipMemsetAsync(scales, 0, static_cast<size_t>(tiles_rows(rows)) * nsq * 512, st));
    const int64_t n = rows * (cols / 8);
    hipLaunchKernelGGL(q4_from_pack_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, pack_dev,
                       rows, cols, codes, scales);
    GV_CHECK_HIP(hipGetLastError());
    out.codes = codes;
    out.scales = scales;
    out.rows = rows;
    out.cols = cols;
    out.S = 0;
    out.steps = 0;
    out.global = global;
    return 0;
}

// ---------------------------------------------------------------- dequant (kernels.cpp:1214-1228)
__global__ void q4_dequant_kernel(Q4 w, float *__restrict__ out) {
    const int64_t nw = w.cols / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= w.rows * nw) return;
    const int64_t r = i / nw, wi = i % nw;
    uint32_t word, sb;
    tq4_word(w, r, wi, word, sb);
    const float s = __fmul_rn(e4m3_to_f32(sb), w.global);   // E4M3 x global, then level x that
    float *o = out + r * w.cols + wi * 8;
    for (int b = 0; b < 8; ++b) {
        const int cp = static_cast<int>((word >> (4 * b)) & 15u);
        o[b] = __fmul_rn(static_cast<float>(2 * cp - 15), s);
    }
}

int q4_dequant(const Q4 &w, float *out, hipStream_t st) {
    const int64_t n = w.rows * (w.cols / 8);
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

// Rows of activations into the products' operands (mfma_gemv.hpp: act16 layout, the int8 path's values), optionally
// RMSNorm first and the normalized fp32 rows out; a workgroup per row.
__global__ __launch_bounds__(256) void quantize_act_kernel(const float *__restrict__ x, int64_t ldx, int cols,
                                                           const float *__restrict__ norm_w, float eps,
                                                           _Float16 *__restrict__ act, int64_t act_stride,
                                                           float *__restrict__ h_out, int64_t ldh) {
    __shared__ double red[16];
    const int t = blockIdx.x;
    norm_quant_row(x + t * ldx, cols, norm_w, eps, act + t * act_stride, h_out ? h_out + t * ldh : nullptr, red);
}

int quantize_act(const float *x, int64_t ldx, int M, int cols, const float *norm_w, float eps, _Float16 *act,
                 int64_t act_stride, float *h_out, int64_t ldh, hipStream_t st) {
    GV_REQUIRE(cols % 16 == 0 && cols <= 8192 && M > 0, "quantize_act: cols must be a multiple of 16, at most 8192");
    GV_REQUIRE(ldx % 4 == 0 && (!h_out || ldh % 4 == 0), "quantize_act: row strides must keep 16-byte alignment");
    hipLaunchKernelGGL(quantize_act_kernel, dim3(M), dim3(256), 0, st, x, ldx, cols, norm_w, eps, act, act_stride,
                       h_out, ldh);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- the skinny GEMM (mfma_gemv.hpp)
// WMAX: the most waves a launch of the instance takes (8: a budget of 256 VGPRs a lane)
// PACK: at most 8 rows, their hi and lo halves in the MFMA's two column halves (mfma_tiles)
// NT > 0 (a launch of at most NT tiles a workgroup): the tile loop straight-line, every tile's loads issued before
// the first tile is computed (NT <= the ring's depth); 0: the ring of three over any number of tiles
// RSPLIT: the M rows in gridDim.y groups of ceil(M / gridDim.y), group blockIdx.y's rows by this workgroup (each row's
// sums as in a launch of its group alone)
template <int KW, int NTT, int WMAX, bool PACK, int NT = 0, bool RSPLIT = false>
__global__ __launch_bounds__(64 * WMAX) void gemv_q4_kernel(Q4 w, const _Float16 *__restrict__ act,
                                                            int64_t act_stride, int M, int sc0, int tiles_per_wg,
                                                            GemvOut out) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    int r0 = 0;   // the first row of the workgroup's group (its outputs' row index offset; out itself is left as
                  // passed: a copy of it would go to scratch, its segment arrays being indexed at run time)
    if constexpr (RSPLIT) {
        const int mh = (M + static_cast<int>(gridDim.y) - 1) / static_cast<int>(gridDim.y);
        r0 = static_cast<int>(blockIdx.y) * mh;
        if (r0 >= M) return;   // (uniform)
        act += static_cast<int64_t>(r0) * act_stride;
        M = min(mh, M - r0);
    }
    const int tc = out.trace_cls;
    if (tc >= 0) trace(tc, 0);
    const int64_t ntiles = tiles_rows(w.rows);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tiles_per_wg;
    const int64_t t1 = t0 + tiles_per_wg < ntiles ? t0 + tiles_per_wg : ntiles;
    if (t0 >= ntiles) return;
    const int nt = static_cast<int>(t1 - t0);
    // The outputs are written as mfma_tiles' split-K epilogue writes them (output o = (tile, column, 4 rows) by
    // thread o mod blockDim), here so that an accumulating product's earlier values for the thread's first output
    // are loaded with the weights (in the hook) rather than one round trip a row at the end.
    const int o0 = threadIdx.x;
    auto item = [&](int o, int64_t &row0, int &j) {
        const int i = o / (NTT * 64), tt = (o / 64) % NTT, ll = o % 64;
        row0 = (t0 + i) * kTileR + 4 * (ll / 16);
        j = tt * 16 + ll % 16;
    };
    float old[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto prefetch = [&] {
        if (!out.accumulate) return;   // uniform
        int64_t row0;
        int j;
        item(min(o0, nt * NTT * 64 - 1), row0, j);
        const float *p = out.y + (r0 + min(j, M - 1)) * out.ldy;
#pragma unroll
        for (int r = 0; r < 4; ++r) old[r] = p[min(row0 + r, w.rows - 1)];   // (clamped: always a valid address)
    };
    mfma_tiles<KW, NTT, kKeepParts, NT, (NT > 0 ? NT : 3), PACK>(
        w.codes, w.scales, w.rows, static_cast<int>(w.cols / kSuperK), sc0, nt, M,
        [&](int j) { return act + j * act_stride; }, [](int64_t, int, float) {}, part_lds, tab, TileRun{t0}, prefetch,
        [&] { if (tc >= 0) trace(tc, 5); });
    if (tc >= 0) trace(tc, 6);
    const int W = blockDim.x / 64;
    for (int o = o0; o < nt * NTT * 64; o += blockDim.x) {   // the waves' partial sums added in wave order
        const int i = o / (NTT * 64), tt = (o / 64) % NTT, ll = o % 64;
        f4 sum = part_lds[((i * W + 0) * NTT + tt) * 64 + ll];
        for (int w2 = 1; w2 < W; ++w2) sum += part_lds[((i * W + w2) * NTT + tt) * 64 + ll];
        int64_t row0;
        int j;
        item(o, row0, j);
        if (j >= M) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = row0 + r;
            if (row >= w.rows) break;
            if (o == o0 && out.accumulate) out.y[(r0 + j) * out.ldy + row] = old[r] + out.scaled(row, sum[r]);
            else out.put(row, r0 + j, sum[r]);
        }
    }
    if (tc >= 0) trace(tc, 3);
}

// The skinny product at 17..32 rows over two K ranges in one launch (each range's activations fill the waves'
// registers, as in two gemv_q4_kernel launches, the second accumulating): the workgroup runs the first range's tiles,
// keeps their partial sums in LDS, runs the second's, then writes (y + s0 x global) + s1 x global (accumulate), or
// s0 x global + s1 x global: the two launches' sums in their order.
template <int KW, int WMAX>
__global__ __launch_bounds__(64 * WMAX) void gemv_q4_2pass_kernel(Q4 w, const _Float16 *__restrict__ act,
                                                                  int64_t act_stride, int M, int sc_step,
                                                                  int tiles_per_wg, GemvOut out) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    const int64_t ntiles = tiles_rows(w.rows);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tiles_per_wg;
    if (t0 >= ntiles) return;
    const int nt = static_cast<int>(std::min<int64_t>(tiles_per_wg, ntiles - t0));
    const int W = blockDim.x / 64, o0 = threadIdx.x;
    f4 *part1 = part_lds + static_cast<size_t>(tiles_per_wg) * W * 2 * 64;
    auto item = [&](int o, int64_t &row0, int &j) {
        const int i = o / 128, tt = (o / 64) % 2, ll = o % 64;
        row0 = (t0 + i) * kTileR + 4 * (ll / 16);
        j = tt * 16 + ll % 16;
    };
    float old[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto prefetch = [&] {
        if (!out.accumulate) return;   // uniform
        int64_t row0;
        int j;
        item(min(o0, nt * 128 - 1), row0, j);
        const float *p = out.y + min(j, M - 1) * out.ldy;
#pragma unroll
        for (int r = 0; r < 4; ++r) old[r] = p[min(row0 + r, w.rows - 1)];   // (clamped: always a valid address)
    };
    const int nsc = static_cast<int>(w.cols / kSuperK);
    mfma_tiles<KW, 2, kKeepParts, 0, 3, false>(w.codes, w.scales, w.rows, nsc, 0, nt, M,
                                                [&](int j) { return act + j * act_stride; },
                                                [](int64_t, int, float) {}, part_lds, tab, TileRun{t0}, prefetch);
    mfma_tiles<KW, 2, kKeepParts, 0, 3, false>(w.codes, w.scales, w.rows, nsc, sc_step, nt, M,
                                                [&](int j) { return act + j * act_stride; },
                                                [](int64_t, int, float) {}, part1, tab, TileRun{t0});
    for (int o = o0; o < nt * 128; o += blockDim.x) {   // each range's waves' partial sums in wave order
        const int i = o / 128, tt = (o / 64) % 2, ll = o % 64;
        f4 s0 = part_lds[((i * W + 0) * 2 + tt) * 64 + ll], s1 = part1[((i * W + 0) * 2 + tt) * 64 + ll];
        for (int w2 = 1; w2 < W; ++w2) {
            s0 += part_lds[((i * W + w2) * 2 + tt) * 64 + ll];
            s1 += part1[((i * W + w2) * 2 + tt) * 64 + ll];
        }
        int64_t row0;
        int j;
        item(o, row0, j);
        if (j >= M) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = row0 + r;
            if (row >= w.rows) break;
            float *p = out.y + j * out.ldy + row;
            const float first = out.scaled(row, s0[r]);
            const float v = out.accumulate ? (o == o0 ? old[r] : *p) + first : first;
            *p = v + out.scaled(row, s1[r]);
        }
    }
}

// The skinny product over many row tiles a workgroup at 17..32 rows (two 16-column tiles: a K range's activations
// take half the registers, so the kept-parts form above holds only 4 tiles' partial sums and each workgroup reloads
// the rows' activations every 4 tiles): the waves' sums put every kGemvFlush tiles (mfma_tiles FLUSH), the same
// sums in the same order as gemv_q4_kernel, so a workgroup takes ~19 tiles with one load of the activations.
constexpr int kGemvFlush = 4;
template <int KW, int WMAX>
__global__ __launch_bounds__(64 * WMAX) void gemv_q4_flush_kernel(Q4 w, const _Float16 *__restrict__ act,
                                                                  int64_t act_stride, int M, int sc0, int tiles_per_wg,
                                                                  GemvOut out) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    const int64_t ntiles = tiles_rows(w.rows);
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tiles_per_wg;
    if (t0 >= ntiles) return;
    const int nt = static_cast<int>(std::min<int64_t>(tiles_per_wg, ntiles - t0));
    mfma_tiles<KW, 2, kSplitK, 0, 3, false, kGemvFlush>(
        w.codes, w.scales, w.rows, static_cast<int>(w.cols / kSuperK), sc0, nt, M,
        [&](int j) { return act + j * act_stride; }, [&](int64_t row, int j, float v) { out.put(row, j, v); },
        part_lds, tab, TileRun{t0});
}

GV_ACT_MODE_SETTER(act_mode_set_q4)
// ---------------------------------------------------------------- the dense SwiGLU FFN (C1) in three launches
// x fp16 rows to the products' operands (the int8 path's quantization of the fp32 values, which fp16 converts to
// exactly): a workgroup a row
__global__ __launch_bounds__(256) void quantize_f16_kernel(const uint16_t *__restrict__ x, int cols,
                                                           _Float16 *__restrict__ act, int64_t act_stride) {
    __shared__ double red[16];
    const int t = blockIdx.x, ng = cols / 8;
    float v[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * blockDim.x;
        uint4 w = make_uint4(0, 0, 0, 0);
        if (g < ng) w = *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(t) * cols + g * 8);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[q][2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u[i] & 0xFFFFu)));
            v[q][2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u[i] >> 16)));
        }
    }
    norm_quant_regs(v, cols, nullptr, 0.0f, act + static_cast<int64_t>(t) * act_stride, nullptr, red);
}

// The gate and up products with the SwiGLU and its quantization in one launch: a workgroup per 16-row tile pair
// (gate tile p, up tile p), its waves splitting K as the skinny product does (the same sums, in the same order); the
// 16 values m = silu(g) x u of a row and tile are one quantization block, so the down product's operands are the
// workgroup's own (at most 8 rows: the rows' hi and lo halves in the MFMA's columns).
template <int KW>
__global__ __launch_bounds__(256) void ffn_up_kernel(Q4 gate, Q4 up, const _Float16 *__restrict__ act,
                                                     int64_t act_stride, int M, _Float16 *__restrict__ act_m,
                                                     int64_t act_m_stride) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    const int p = blockIdx.x, W = blockDim.x / 64, lane = threadIdx.x % 64;
    const int nsc = static_cast<int>(gate.cols / kSuperK);
    auto rowp = [&](int j) { return act + static_cast<int64_t>(min(j, M - 1)) * act_stride; };
    auto tile = [&](int) -> int64_t { return p; };
    mfma_tiles<KW, 1, kKeepParts, 1, 2, true>(gate.codes, gate.scales, gate.rows, nsc, 0, 1, M, rowp,
                                              [](int64_t, int, float) {}, part_lds, tab, tile);
    mfma_tiles<KW, 1, kKeepParts, 1, 2, true>(up.codes, up.scales, up.rows, nsc, 0, 1, M, rowp,
                                              [](int64_t, int, float) {}, part_lds + W * 64, tab, tile);
    if (threadIdx.x >= 64) return;
    // the waves' sums in wave order x global (the products' put), m = silu(g) x u (swiglu's arithmetic), the block's
    // operands (quantize_activation); lane (j = lane % 16, lg = lane / 16): rows 4 lg .. 4 lg + 3 of the tile, row j
    const int j = lane % 16, lg = lane / 16;
    f4 gs = part_lds[lane], us = part_lds[W * 64 + lane];
    for (int w2 = 1; w2 < W; ++w2) {
        gs += part_lds[w2 * 64 + lane];
        us += part_lds[(W + w2) * 64 + lane];
    }
    float mv[4], amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = gs[r] * gate.global, uv = us[r] * up.global;
        mv[r] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), uv);
        amax = fmaxf(amax, fabsf(mv[r]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float sc = __fdiv_rn(amax, 127.0f), qi = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    uint32_t hw[2], lw[2];
#pragma unroll
    for (int r = 0; r < 4; r += 2) {
        _Float16 h0, l0, h1, l1;
        const int q0 = min(max(static_cast<int>(rintf(__fmul_rn(mv[r], qi))), -127), 127);
        const int q1 = min(max(static_cast<int>(rintf(__fmul_rn(mv[r + 1], qi))), -127), 127);
        const bool ex = g_act_exact != 0;   // (the exact path: the SwiGLU values themselves)
        split_f16(ex ? mv[r] : __fmul_rn(static_cast<float>(q0), sc), h0, l0);
        split_f16(ex ? mv[r + 1] : __fmul_rn(static_cast<float>(q1), sc), h1, l1);
        hw[r / 2] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h0)) |
                    (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
        lw[r / 2] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l0)) |
                    (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
    }
    // k-group 2 p + lg / 2 holds values 0..3 (lane lg even) and 4..7 (lane lg + 1) in the slot order
    // (0 4 1 5 2 6 3 7): the even lane takes its partner's four and writes the group
    uint32_t ph[2], pl[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        ph[k] = __shfl_xor(hw[k], 16, 64);
        pl[k] = __shfl_xor(lw[k], 16, 64);
    }
    if ((lg & 1) == 0 && j < M) {
        auto inter = [](uint32_t mine, uint32_t other) {
            return make_uint2((mine & 0xFFFFu) | (other << 16), (mine >> 16) | (other & 0xFFFF0000u));
        };
        const uint2 h01 = inter(hw[0], ph[0]), h23 = inter(hw[1], ph[1]);
        const uint2 l01 = inter(lw[0], pl[0]), l23 = inter(lw[1], pl[1]);
        uint4 *dst = reinterpret_cast<uint4 *>(act_m + j * act_m_stride + static_cast<int64_t>(2 * p + lg / 2) * 16);
        dst[0] = make_uint4(h01.x, h01.y, h23.x, h23.y);
        dst[1] = make_uint4(l01.x, l01.y, l23.x, l23.y);
    }
}

int quantize_f16(const uint16_t *x, int M, int cols, _Float16 *act, int64_t act_stride, hipStream_t st) {
    GV_REQUIRE(cols % 16 == 0 && cols <= 8192 && M > 0, "quantize_f16: cols must be a multiple of 16, at most 8192");
    hipLaunchKernelGGL(quantize_f16_kernel, dim3(M), dim3(256), 0, st, x, cols, act, act_stride);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int ffn_up(const Q4 &gate, const Q4 &up, const _Float16 *act, int64_t act_stride, int M, _Float16 *act_m,
           int64_t act_m_stride, hipStream_t st) {
    int waves = 0, kw = 0;
    GV_REQUIRE(M >= 1 && M <= 8 && gate.rows == up.rows && gate.cols == up.cols && gate.rows % kTileR == 0 &&
                   mfma_split(gate.cols, 1, waves, kw) && waves <= 4,
               "ffn_up: 1 <= M <= 8, gate and up alike, whole row tiles, K split over at most 4 waves");
    const dim3 grid(static_cast<unsigned>(gate.rows / kTileR)), block(static_cast<unsigned>(64 * waves));
    const size_t lds = static_cast<size_t>(2 * waves) * 1024;
    if (kw == 16) hipLaunchKernelGGL(ffn_up_kernel<16>, grid, block, lds, st, gate, up, act, act_stride, M, act_m, act_m_stride);
    else if (kw == 8) hipLaunchKernelGGL(ffn_up_kernel<8>, grid, block, lds, st, gate, up, act, act_stride, M, act_m, act_m_stride);
    else hipLaunchKernelGGL(ffn_up_kernel<4>, grid, block, lds, st, gate, up, act, act_stride, M, act_m, act_m_stride);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}


int trace_set_q4(uint64_t *p) {
    GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &p, sizeof p));
    return 0;
}

int mfma_split(int64_t K, int ntt, int &waves, int &kw) {
    const int chunks = static_cast<int>(K / 32);
    kw = ntt == 1 ? 16 : 8;
    while (kw > 4 && (chunks % kw || chunks / kw < 2)) kw /= 2;
    waves = chunks / kw;
    return K % kSuperK == 0 && waves >= 1 && waves <= 8;
}

// tiles a workgroup: about as many workgroups as the chip holds at once (2 waves a SIMD at these kernels' register
// use: 512 / waves workgroups), the waves' partial sums within 76 KB of LDS (two workgroups a CU)
int64_t tiles_per_wg(int64_t ntiles, int waves, int ntt) {
    const int64_t resident = 256 * std::max(1, 8 / waves);
    const int64_t cap = waves > 1 ? std::max(1, 76 / (waves * ntt)) : 64;
    return std::min<int64_t>(cap, std::max<int64_t>(1, (ntiles + resident - 1) / resident));
}

template <int KW, int NTT, int WMAX, bool PACK>
static int launch_gemv(const Q4 &w, const _Float16 *act, int64_t act_stride, int M, int sc0, int waves,
                       const GemvOut &out, hipStream_t st) {
    const int64_t ntiles = tiles_rows(w.rows);
    const int64_t per = tiles_per_wg(ntiles, waves, NTT);
    if constexpr (NTT == 2 && !PACK) {
        // a matrix whose tiles outnumber 4 a workgroup of the chip's resident ones (the head at a tree's 17 rows):
        // the flushed form, ~2 workgroups a CU's worth of tiles each
        const int64_t resident = 256 * std::max(1, 8 / waves);
        if (ntiles > per * resident) {
            const int64_t pf = std::max<int64_t>(kGemvFlush, (ntiles + 2 * resident - 1) / (2 * resident));
            const int64_t wgf = (ntiles + pf - 1) / pf;
            const size_t ldsf = static_cast<size_t>(kGemvFlush) * waves * NTT * 1024;
            static int granted_f = 0;
            if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_flush_kernel<KW, WMAX>), 76 * 1024, granted_f) != 0)
                return -1;
            hipLaunchKernelGGL((gemv_q4_flush_kernel<KW, WMAX>), dim3(static_cast<unsigned>(wgf)), dim3(64 * waves), ldsf,
                               st, w, act, act_stride, M, sc0, static_cast<int>(pf), out);
            return 0;
        }
    }
    const int64_t wg = (ntiles + per - 1) / per;
    const size_t lds = static_cast<size_t>(per) * waves * NTT * 1024;   // the waves' partial sums
    if (per <= 3 && per > 1) {   // a few tiles a workgroup (q|k|v): all of them in flight at once
        static int granted3 = 0;
        if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_kernel<KW, NTT, WMAX, PACK, 3>), 76 * 1024, granted3) != 0)
            return -1;
        hipLaunchKernelGGL((gemv_q4_kernel<KW, NTT, WMAX, PACK, 3>), dim3(static_cast<unsigned>(wg)), dim3(64 * waves),
                           static_cast<size_t>(3) * waves * NTT * 1024, st, w, act, act_stride, M, sc0,
                           static_cast<int>(per), out);
        return 0;
    }
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_kernel<KW, NTT, WMAX, PACK>), 76 * 1024, granted) != 0)
        return -1;
    hipLaunchKernelGGL((gemv_q4_kernel<KW, NTT, WMAX, PACK>), dim3(static_cast<unsigned>(wg)), dim3(64 * waves), lds,
                       st, w, act, act_stride, M, sc0, static_cast<int>(per), out);
    return 0;
}

// one launch over super-chunks [sc0, sc0 + n) of every row
static int gemv_range(const Q4 &w, const _Float16 *act, int64_t act_stride, int M, int ntt, int sc0, int n,
                      const GemvOut &out, hipStream_t st) {
    int waves, kw;
    if (!mfma_split(static_cast<int64_t>(n) * kSuperK, ntt, waves, kw)) {
        set_error("gemv_q4: no split of this K range");
        return -1;
    }
    // a short launch (a few tiles a workgroup): eight waves, each half the decode chain (measured: the 9216-row
    // q|k|v product 9.6 -> 8.3 us; the 151,936-row lm_head keeps four, 36.8 against 39.9 us)
    if (ntt == 1 && waves <= 4 && kw == 16 && tiles_rows(w.rows) < 2048) kw = 8, waves *= 2;
    if (ntt == 1 && M <= 8) {
        if (kw == 16) return launch_gemv<16, 1, 8, true>(w, act, act_stride, M, sc0, waves, out, st);
        if (kw == 8) return launch_gemv<8, 1, 8, true>(w, act, act_stride, M, sc0, waves, out, st);
        return launch_gemv<4, 1, 8, true>(w, act, act_stride, M, sc0, waves, out, st);
    }
    if (ntt == 1) {
        if (kw == 16) return launch_gemv<16, 1, 8, false>(w, act, act_stride, M, sc0, waves, out, st);
        if (kw == 8) return launch_gemv<8, 1, 8, false>(w, act, act_stride, M, sc0, waves, out, st);
        return launch_gemv<4, 1, 8, false>(w, act, act_stride, M, sc0, waves, out, st);
    }
    if (kw == 8) return launch_gemv<8, 2, 8, false>(w, act, act_stride, M, sc0, waves, out, st);
    return launch_gemv<4, 2, 8, false>(w, act, act_stride, M, sc0, waves, out, st);
}

int gemv_q4(const Q4 &w, const _Float16 *act, int64_t act_stride, int M, const GemvOut &out, hipStream_t st) {
    GV_REQUIRE(M >= 1 && M <= kMaxRows, "gemv_q4: 1 <= M <= 32 rows");
    GV_REQUIRE(w.cols % kSuperK == 0 && w.cols <= kMaxActCols, "gemv_q4: cols must be a multiple of 128, at most 16384");
    const int ntt = M <= 16 ? 1 : 2;
    const int nsc = static_cast<int>(w.cols / kSuperK);
    if (ntt == 2 && nsc == 32) {   // 17..32 rows over K = 4096 (the tree's output projection), a few tiles: the rows in
                                   // two groups of at most 16, each over the whole K in one range (the sums of an
                                   // M <= 16 launch), both groups in one launch: twice the workgroups, each loading
                                   // half the rows' operands
        int waves, kw;
        const int64_t ntiles = tiles_rows(w.rows);
        if (mfma_split(32 * kSuperK, 1, waves, kw) && kw == 16 && waves == 8 && tiles_per_wg(ntiles, waves, 1) == 1) {
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_kernel<16, 1, 8, false, 0, true>), 76 * 1024,
                          granted) != 0)
                return -1;
            hipLaunchKernelGGL((gemv_q4_kernel<16, 1, 8, false, 0, true>), dim3(static_cast<unsigned>(ntiles), 2),
                               dim3(64 * waves), static_cast<size_t>(waves) * 1024, st, w, act, act_stride, M, 0, 1,
                               out);
            GV_CHECK_HIP(hipGetLastError());
            return 0;
        }
    }
    // K ranges whose activations fit the waves' registers: one launch up to 4096 (2048 for 17..32 rows) values,
    // later ranges adding to the first's sums
    if (ntt == 2 && nsc == 32) {   // two ranges of 2048 in one launch (kept parts, up to two tiles a workgroup)
        int waves, kw;
        const int64_t ntiles = tiles_rows(w.rows);
        if (mfma_split(16 * kSuperK, 2, waves, kw) && kw == 8 && waves == 8 && tiles_per_wg(ntiles, waves, 2) <= 2) {
            const int64_t per = tiles_per_wg(ntiles, waves, 2), wg = (ntiles + per - 1) / per;
            const size_t lds = static_cast<size_t>(2 * per) * waves * 2 * 1024;
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&gemv_q4_2pass_kernel<8, 8>), lds, granted) != 0) return -1;
            hipLaunchKernelGGL((gemv_q4_2pass_kernel<8, 8>), dim3(static_cast<unsigned>(wg)), dim3(64 * waves), lds, st,
                               w, act, act_stride, M, 16, static_cast<int>(per), out);
            GV_CHECK_HIP(hipGetLastError());
            return 0;
        }
    }
    for (int sc0 = 0, part = 0; sc0 < nsc; ++part) {
        int n = std::min(nsc - sc0, ntt == 1 ? 32 : 16);
        int waves, kw;
        while (n > 1 && !mfma_split(static_cast<int64_t>(n) * kSuperK, ntt, waves, kw)) --n;
        GV_REQUIRE(sc0 % 4 == 0, "gemv_q4: a K range must start on a quad of super-chunks");
        GemvOut o = out;
        if (part > 0) o.accumulate = 1;
        if (gemv_range(w, act, act_stride, M, ntt, sc0, n, o, st) != 0) return -1;
        sc0 += n;
    }
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace gv
