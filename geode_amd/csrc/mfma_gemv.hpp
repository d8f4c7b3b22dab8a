// mfma_gemv.hpp - the skinny products on the matrix cores (v_mfma_f32_16x16x32_f16).
//
// y[t][r] = sum_k W[r][k] x[t][k] for up to 32 rows t of activations. The weights are the q4 matrix's exact values
// level x E4M3(scale) (at most 8 significant bits: exact in fp16), made in registers from the nibbles; global is
// applied to the fp32 sums. The activations are staged as two fp16 halves hi + lo of their fp32 value (hi + lo =
// the value to 2^-22), so each product is two MFMAs and the result is the fp32 one up to summation order. On the
// int8 path (the reference's default, matvec_rows_q_ref in engine/src/kernels.cpp:1304-1322) the activation value
// is its int8 code times its block scale, q x (amax / 127): the same products as the integer block sums times the
// block scales.
//
// The q4 layout of these kernels ("tiles"): rows in tiles of 16, K in super-chunks of 128 values. A tile's
// super-chunk is 1 KB of codes: lane l (row l % 16, k-group g = l / 16) has 16 bytes = the pack's code words
// 16 sc + 4 j + g (j = 0..3: the 32-value chunks of the super-chunk, 8 values of the k-group each), nibbles remapped
// to the affine order (level = 2c' - 15) and placed for decode8 (tile_word). One load instruction of a wave reads the
// 1 KB whole. The E4M3 scales apart, per tile and per quad of four super-chunks (sc = 4 q + s), 512 bytes: byte
// ((r * 2 + g / 2) * 4 + s) * 4 + j = the block of chunk j of super-chunk sc that k-group g falls in, so a lane's
// words of the quad's four super-chunks are one 16-byte load (tq4_scale_off).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace gv {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kTileR = 16;    // rows a tile
constexpr int kSuperK = 128;  // values a super-chunk

__host__ __device__ inline int64_t tiles_rows(int64_t rows) { return (rows + kTileR - 1) / kTileR; }
inline size_t tq4_code_bytes(int64_t rows, int64_t cols) { return static_cast<size_t>(tiles_rows(rows)) * kTileR * (cols / 2); }
inline size_t tq4_scale_bytes(int64_t rows, int64_t cols) { return static_cast<size_t>(tiles_rows(rows)) * ((cols / kSuperK + 3) / 4) * 512; }
// the byte of the scale of (tile T, super-chunk sc, row r of the tile, k-group g, chunk j); nsq = quads a tile row
__host__ __device__ inline int64_t tq4_scale_off(int64_t T, int64_t nsq, int64_t sc, int64_t r, int64_t g, int64_t j) {
    return (T * nsq + sc / 4) * 512 + ((r * 2 + g / 2) * 4 + sc % 4) * 4 + j;
}

// The activations' layout for these kernels: per row, per k-group g (values 8 g .. 8 g + 7; chunk g / 4, k-group g % 4
// of it), 8 hi halves then 8 lo halves (32 bytes) of values 8 g + (0 4 1 5 2 6 3 7), the order the nibble pairs come
// out in.
inline size_t act16_row_bytes(int64_t cols) { return static_cast<size_t>(cols) * 4; }

// One k-group's operands: v = values 8 g .. 8 g + 7 of a row, the int8 path's q x (amax / 127) (quantize_activation,
// engine/src/kernels.cpp:1254-1295, bit for bit) written as hi + lo halves at the group's 32 bytes. The 16-value
// block is the groups g and g ^ 1, held by lanes l and l ^ 1: every lane of the wave calls this (live = false: a lane
// past the row's end, which stores nothing).
// The products' operands are the int8 path's values (0, the reference's default) or the fp32 values themselves (1:
// the exact path, ModelOptions::exact, engine/src/model.cpp:3337-3361 with kernels.cpp:1230-1250: fp32 activations
// against the dequantized weights), both written as hi + lo halves (hi + lo = the value to 2^-22). Each source
// file's kernels read their own copy; the act_mode_set_* functions set them (between launches only).
static __constant__ int g_act_exact;
#define GV_ACT_MODE_SETTER(name)                                                   \
    int name(int exact) {                                                          \
        GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_act_exact), &exact, sizeof exact)); \
        return 0;                                                                  \
    }

// 8 values of a 16-value block with the block's amax into their operands: q x (amax / 127) (the exact path: the
// values) as hi + lo halves in the slot order (0 4 1 5 2 6 3 7)
__device__ inline void act16_operands(const float (&v)[8], float amax, h8 &hi, h8 &lo) {
    if (g_act_exact) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int slot = i < 4 ? 2 * i : 2 * (i - 4) + 1;
            _Float16 yh, yl;
            split_f16(v[i], yh, yl);
            hi[slot] = yh;
            lo[slot] = yl;
        }
        return;
    }
    const float s = __fdiv_rn(amax, 127.0f), qi = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = min(max(static_cast<int>(rintf(__fmul_rn(v[i], qi))), -127), 127);
        const float y = __fmul_rn(static_cast<float>(q), s);
        const int slot = i < 4 ? 2 * i : 2 * (i - 4) + 1;
        _Float16 yh, yl;
        split_f16(y, yh, yl);
        hi[slot] = yh;
        lo[slot] = yl;
    }
}

__device__ inline float amax8(const float (&v)[8]) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
    return a;
}

__device__ inline void act16_store(_Float16 *ar, int g, bool live, const h8 &hi, const h8 &lo) {
    if (!live) return;
    h8 *p = reinterpret_cast<h8 *>(ar + static_cast<int64_t>(g) * 16);
    p[0] = hi;
    p[1] = lo;
}
template <typename Dst>
__device__ inline void act16_group(const float (&v)[8], int g, bool live, Dst ar) {
    const float amax = fmaxf(amax8(v), __shfl_xor(amax8(v), 1, 64));
    h8 hi, lo;
    act16_operands(v, amax, hi, lo);
    act16_store(ar, g, live, hi, lo);
}

// A row of cols (a multiple of 16, at most 32 blockDim) values, held in registers, into its operands: thread i has
// the 8-value groups i, i + blockDim, ... (up to 4; zeros past the row), optionally RMSNorm(1 + w) first (rmsnorm's
// arithmetic, engine/src/kernels.cpp:1520-1529: the double sum of squares, inv = 1 / sqrt(float(ss / n) + eps), x inv
// (1 + w)) and the normalized fp32 row to h (if not null). The whole workgroup calls this; red: LDS of 16 doubles.
// the thread's norm weights 1 + w of its groups (as norm_quant_regs takes them), loaded ahead of their use
__device__ inline void norm_weights(const float *norm_w, int cols, float (&w1)[4][8]) {
    const int ng = cols / 8, nthr = blockDim.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * nthr;
        float4 a = make_float4(0, 0, 0, 0), b = a;
        if (norm_w && g < ng) {
            a = *reinterpret_cast<const float4 *>(norm_w + g * 8);
            b = *reinterpret_cast<const float4 *>(norm_w + g * 8 + 4);
        }
        const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) w1[q][i] = __fadd_rn(1.0f, t[i]);
    }
}

// norm_quant_regs with the norm weights already in registers (has_norm false: no norm)
template <typename Dst>
__device__ inline void norm_quant_regs_w(float (&v)[4][8], int cols, bool has_norm, const float (&w1)[4][8],
                                         float eps, Dst ar, float *h, double *red);

template <typename Dst>
__device__ inline void norm_quant_regs(float (&v)[4][8], int cols, const float *norm_w, float eps, Dst ar,
                                       float *h, double *red) {
    float w1[4][8];
    if (norm_w) norm_weights(norm_w, cols, w1);
    norm_quant_regs_w(v, cols, norm_w != nullptr, w1, eps, ar, h, red);
}

template <typename Dst>
__device__ inline void norm_quant_regs_w(float (&v)[4][8], int cols, bool has_norm, const float (&w1)[4][8],
                                         float eps, Dst ar, float *h, double *red) {
    const int ng = cols / 8, nthr = blockDim.x;
    if (has_norm) {
        double ss = 0.0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += static_cast<double>(v[q][i]) * static_cast<double>(v[q][i]);
        ss = wave_sum(ss);
        __syncthreads();   // red may still be read by an earlier call
        if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = ss;
        __syncthreads();
        double tot = 0.0;
        for (int w = 0; w < nthr / 64; ++w) tot += red[w];
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(cols)), eps)));
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[q][i] = __fmul_rn(__fmul_rn(v[q][i], inv), w1[q][i]);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (q * nthr >= ng) break;   // uniform: no lane has a group from here on
        const int g = threadIdx.x + q * nthr;
        const bool live = g < ng;
        if (h && live) {
            *reinterpret_cast<float4 *>(h + g * 8) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
            *reinterpret_cast<float4 *>(h + g * 8 + 4) = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
        }
        act16_group(v[q], g, live, ar);
    }
}

// norm_quant_regs of a row in memory (global or LDS, 16-byte aligned), loaded once
__device__ inline void norm_quant_row(const float *x, int cols, const float *norm_w, float eps, _Float16 *ar, float *h,
                                      double *red) {
    const int ng = cols / 8;
    float v[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * blockDim.x;
        float4 a = make_float4(0, 0, 0, 0), b = a;
        if (g < ng) {
            a = *reinterpret_cast<const float4 *>(x + g * 8);
            b = *reinterpret_cast<const float4 *>(x + g * 8 + 4);
        }
        const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[q][i] = t[i];
    }
    norm_quant_regs(v, cols, norm_w, eps, ar, h, red);
}

// Where a code word's nibbles sit. decode8 makes the A operand's pairs (v_i, v_i+4), i = 0..3, from 4 views of the
// word (itself, << 4, >> 4, rotated right by 8); in view i the pair's nibbles sit at bits 6..9 and 22..25. tile_word
// places the 8 affine codes of a word (nibble i = value i) so, untile_word takes them back.
__host__ __device__ inline uint32_t tile_word(uint32_t a) {
    uint32_t p[4];
    for (int i = 0; i < 4; ++i) p[i] = (((a >> (4 * i)) & 15u) << 6) | (((a >> (4 * i + 16)) & 15u) << 22);
    return p[0] | (p[1] >> 4) | (p[2] << 4) | (p[3] << 8) | (p[3] >> 24);
}
__host__ __device__ inline uint32_t untile_word(uint32_t w) {
    const uint32_t d[4] = {w, w << 4, w >> 4, (w >> 8) | (w << 24)};
    uint32_t a = 0;
    for (int i = 0; i < 4; ++i) a |= (((d[i] >> 6) & 15u) << (4 * i)) | (((d[i] >> 22) & 15u) << (4 * i + 16));
    return a;
}

// code word wi (values 8 wi .. 8 wi + 7) of row r of a tile-layout matrix: the 8 affine codes (nibble i = value i)
// and the block's scale byte
__device__ inline void tq4_word(const Q4 &w, int64_t r, int64_t wi, uint32_t &word, uint32_t &scale) {
    const int64_t T = r / kTileR, rr = r % kTileR, nsc = w.cols / kSuperK;
    const int64_t sc = wi / 16, j = (wi % 16) / 4, g = wi % 4;
    const int64_t blk = T * nsc + sc;
    word = untile_word(*reinterpret_cast<const uint32_t *>(w.codes + blk * 1024 + (rr + 16 * g) * 16 + j * 4));
    scale = w.scales[tq4_scale_off(T, (nsc + 3) / 4, sc, rr, g, j)];
}

// The scale table: per E4M3 byte, the fp16 pairs (e4 / 32, -47 e4). With a nibble c' at bits 6..9 of the fp16
// 1024.0 (0x6400), v = 1024 + 64 c' and fma(v, e4 / 32, -47 e4) = (2 c' - 15) e4 = level x E4M3, exactly: v x e4 / 32
// is exact inside the fma, -47 e4 has at most 10 significant bits, and the result at most 8 (all E4M3 values,
// subnormals included, stay fp16 normals here).
__device__ inline void fill_e4m3_table(uint2 *tab) {
    for (int b = threadIdx.x; b < 256; b += blockDim.x) {
        const float e = e4m3_to_f32(static_cast<uint32_t>(b));
        const uint32_t m = __builtin_bit_cast(uint16_t, static_cast<_Float16>(e * 0.03125f));
        const uint32_t c = __builtin_bit_cast(uint16_t, static_cast<_Float16>(-47.0f * e));
        tab[b] = make_uint2(m | (m << 16), c | (c << 16));
    }
}

// (x & mask) | magic in one instruction (mask from a scalar register, magic from a vector one)
__device__ inline uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(magic));
    return r;
}

// 8 weights of one code word as the A operand, level x E4M3 each in fp16: pairs (v_i, v_i+4), i = 0..3
__device__ inline h8 decode8(uint32_t w, uint2 sc, uint32_t magic) {
    const uint32_t d[4] = {w, w << 4, w >> 4, __builtin_amdgcn_alignbit(w, w, 8)};
    const h2 m = __builtin_bit_cast(h2, sc.x), c = __builtin_bit_cast(h2, sc.y);
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 v = __builtin_bit_cast(h2, and_or(d[i], 0x03C003C0u, magic));
        r[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(v, m, c));
    }
    return __builtin_bit_cast(h8, make_uint4(r[0], r[1], r[2], r[3]));
}

// the operands of k-group g of an act16 row
__device__ inline void load_act16(const _Float16 *ar, int64_t g, h8 &hi, h8 &lo) {
    const _Float16 *p = ar + g * 16;
    hi = *reinterpret_cast<const h8 *>(p);
    lo = *reinterpret_cast<const h8 *>(p + 8);
}

// An act16 row of zeros for the operand rows past M (64 KB: rows of up to 16,384 values): loading zeros instead of
// zeroing the registers after a load keeps the compiler from waiting for every load in flight before the first tile
static __device__ uint4 g_zero_act16[4096];
constexpr int64_t kMaxActCols = 16384;

// The tiles a call takes: local tile i is tile t0 + i of the matrix (a run), or any map i -> tile
struct TileRun {
    int64_t t0;
    __device__ int64_t operator()(int i) const { return t0 + i; }
};
struct NoHook {
    __device__ void operator()() const {}
};
// a call's own output of the flushed tiles (mfma_tiles, kSplitK with FLUSH): flush(i0, i1, part, W) takes tiles
// [i0, i1)'s waves' partial sums (part[((i - i0) W + w) NTT + tt) 64 + lane]) instead of put; active false: put
struct NoFlush {
    static constexpr bool active = false;
    __device__ void operator()(int, int, const f4 *, int) const {}
};
template <typename F>
struct FlushWith {
    static constexpr bool active = true;
    F f;
    __device__ void operator()(int i0, int i1, const f4 *part, int W) const { f(i0, i1, part, W); }
};
template <typename F>
__device__ inline FlushWith<F> flush_with(F f) { return FlushWith<F>{f}; }

// How a call's waves share the work: kSplitK - the workgroup's waves split the K range of every tile, their partial
// sums added in wave order at the end (then put); kKeepParts - the same, the partial sums left in LDS for the caller;
// kWaveTiles - each wave alone over the whole K range and its own tiles, put directly.
enum TilesMode { kSplitK = 0, kKeepParts = 1, kWaveTiles = 2 };

// One share of a product: W waves split the K range [sc0, sc0 + W KW / 4) super-chunks (wave w: chunks
// [w KW, (w + 1) KW) of it) of nt row tiles (local tile i is tile tmap(i)), a tile at a time with the next DEPTH - 1
// tiles' loads in flight; nsc = super-chunks a row (W = 1 in kWaveTiles). NT > 0: nt <= NT, and the tile loop is
// unrolled NT times (straight-line code: the compiler then waits for exactly the loads a tile needs; tiles past nt
// are computed on the last tile's data and dropped); NT = 0: a runtime loop. rowp(j) is local row j's act16 operands
// (any j < M). PACK (M <= 8, NTT = 1): the MFMA's 16 columns hold the rows' hi halves (columns 0..7) and their lo
// halves (8..15), so one MFMA chain makes both products (each column's sum is the one the unpacked form makes) and a
// lane swap adds them; else the hi and lo halves are two chains. put(row, j, v) takes the fp32 sum (before global).
// part: LDS of max(nt, NT) * W * NTT KB for the waves' partial sums (kSplitK, kKeepParts: part[((i W + w) NTT + tt)
// 64 + lane], left there after a workgroup barrier in kKeepParts); FLUSH > 0 (kSplitK, runtime loop): the sums of
// every FLUSH tiles are put as soon as those tiles are done, so part holds FLUSH * W * NTT KB whatever nt is (the
// activations stay in registers over many tiles); tab: LDS for fill_e4m3_table, filled here. hook()
// runs after the first tiles' loads are issued and before the activations are loaded (a wait for them); ready() once
// the activations and the first tiles are in registers. Every thread of the workgroup calls this.
template <int KW, int NTT, int MODE, int NT = 0, int DEPTH = 3, bool PACK = false, int FLUSH = 0, typename RowFn,
          typename PutFn, typename MapFn = TileRun, typename HookFn = NoHook, typename ReadyFn = NoHook,
          typename FlushFn = NoFlush>
__device__ inline void mfma_tiles(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, int64_t rows,
                                  int nsc, int sc0, int nt, int M, RowFn rowp, PutFn put, f4 *part, uint2 *tab,
                                  MapFn tmap, HookFn hook = HookFn{}, ReadyFn ready = ReadyFn{},
                                  FlushFn flush = FlushFn{}) {
    static_assert(DEPTH >= 2 && (NT > 0 || DEPTH >= 3), "the runtime loop is a ring of at least three");
    static_assert(!PACK || NTT == 1, "packed hi | lo columns take one 16-row tile of at most 8 rows");
    static_assert(FLUSH == 0 || (MODE == kSplitK && NT == 0), "the flushed split-K runs the runtime tile loop");
    constexpr int NB = PACK ? 1 : 2;   // operand arrays: hi | lo packed, or hi and lo
    const int W = MODE == kWaveTiles ? 1 : static_cast<int>(blockDim.x / 64);
    const int w = MODE == kWaveTiles ? 0 : static_cast<int>(threadIdx.x / 64);
    const int l = threadIdx.x % 64, lq = l % 16, lg = l / 16;
    constexpr int NS = KW / 4;   // super-chunks a wave takes
    const uint32_t magic = 0x64006400u;
    const uint8_t *cbase = codes + static_cast<int64_t>(sc0 + w * NS) * 1024 + l * 16;
    // the lane's scale words of its NS super-chunks: adjacent in one quad (sc0 a multiple of 4, NS = 1, 2 or 4)
    const uint32_t nsq_u = static_cast<uint32_t>((nsc + 3) / 4);
    const uint8_t *sbase =
        scales + static_cast<int64_t>((sc0 + w * NS) / 4) * 512 + ((lq * 2 + lg / 2) * 4 + (sc0 + w * NS) % 4) * 4;
    // Every load is issued unconditionally (a tile past nt reads the last tile again, from the cache): a branch
    // around a load makes the compiler wait for nearly all loads in flight before the next use. Offsets in 32 bits
    // (a matrix < 4 GB).
    const uint32_t nsc_u = static_cast<uint32_t>(nsc);
    auto load = [&](int i, uint4 (&cw)[NS], uint32_t (&sw)[NS]) {
        const uint32_t T = nt > 0 ? static_cast<uint32_t>(tmap(i < nt ? i : nt - 1)) : 0u;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t blk = T * nsc_u + static_cast<uint32_t>(s);
            const u4v v = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(cbase + blk * 1024u));
            cw[s] = make_uint4(v.x, v.y, v.z, v.w);
        }
        const uint8_t *sp = sbase + T * nsq_u * 512u;
        if constexpr (NS == 4) {
            const u4v v = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(sp));
            sw[0] = v.x, sw[1] = v.y, sw[2] = v.z, sw[3] = v.w;
        } else if constexpr (NS == 2) {
            typedef uint32_t u2v __attribute__((ext_vector_type(2)));
            const u2v v = __builtin_nontemporal_load(reinterpret_cast<const u2v *>(sp));
            sw[0] = v.x, sw[1] = v.y;
        } else {
            sw[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(sp));
        }
    };
    // the first two tiles' weights (HBM, the longest wait) first, then the activations, then the rest of the
    // prologue's tiles: loads complete in issue order, so the first tile waits for two tiles and the activations only
    constexpr int PRE = DEPTH - 1 < 2 ? DEPTH - 1 : 2;
    uint4 cw[DEPTH][NS];
    uint32_t sw[DEPTH][NS];
#pragma unroll
    for (int d = 0; d < PRE; ++d) load(d, cw[d], sw[d]);
    hook();
    // the activations of this wave's K range, resident for all the tiles (rows past M: zeros)
    h8 b[NB][KW][NTT];
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const int j = PACK ? lq % 8 : tt * 16 + lq;
        const _Float16 *row = j < M ? rowp(j) : reinterpret_cast<const _Float16 *>(g_zero_act16);
#pragma unroll
        for (int c = 0; c < KW; ++c) {
            const int64_t g = (static_cast<int64_t>(sc0) * 4 + w * KW + c) * 4 + lg;
            if (PACK) {
                b[0][c][tt] = *reinterpret_cast<const h8 *>(row + g * 16 + (lq >= 8 ? 8 : 0));
            } else {
                b[0][c][tt] = *reinterpret_cast<const h8 *>(row + g * 16);
                b[NB - 1][c][tt] = *reinterpret_cast<const h8 *>(row + g * 16 + 8);
            }
        }
    }
#pragma unroll
    for (int d = PRE; d < DEPTH - 1; ++d) load(d, cw[d], sw[d]);
    fill_e4m3_table(tab);
    __syncthreads();
    auto tile = [&](int i, const uint4 (&cq)[NS], const uint32_t (&sq)[NS]) {
        f4 acc[NB][NTT];   // the hi and lo products apart: two independent MFMA chains (packed: two column halves)
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
            for (int h = 0; h < NB; ++h) acc[h][tt] = f4{0, 0, 0, 0};
        uint2 tv[NS][4];   // the tile's scale table entries, all read from the LDS before the first is used
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) tv[s][j] = tab[(sq[s] >> (8 * j)) & 0xFFu];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const uint32_t words[4] = {cq[s].x, cq[s].y, cq[s].z, cq[s].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const h8 a = decode8(words[j], tv[s][j], magic);
                const int c = s * 4 + j;
#pragma unroll
                for (int tt = 0; tt < NTT; ++tt)
#pragma unroll
                    for (int h = 0; h < NB; ++h)
                        acc[h][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[h][c][tt], acc[h][tt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
            if (PACK) {   // column j < 8: hi sum + the lo sum from column j + 8 (lane l ^ 8)
                f4 lo;
#pragma unroll
                for (int r = 0; r < 4; ++r) lo[r] = xor8(acc[0][tt][r]);
                acc[0][tt] += lo;
            } else {
                acc[0][tt] += acc[NB - 1][tt];
            }
        }
        f4 (&res)[NTT] = acc[0];
        if (MODE != kWaveTiles) {
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) part[(((FLUSH ? i % FLUSH : i) * W + w) * NTT + tt) * 64 + l] = res[tt];
        } else if (i < nt) {
            const int64_t T = tmap(i);
#pragma unroll
            for (int tt = 0; tt < NTT; ++tt) {
                const int j = tt * 16 + lq;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = T * kTileR + 4 * lg + r;
                    if (j < M && row < rows) put(row, j, res[tt][r]);
                }
            }
        }
    };
    // the waves' partial sums of tiles [i0, i1) (at i - i0 in part, or i when every tile's are kept) added in wave
    // order, each output by one thread
    auto split_k_out = [&](int i0, int i1) {
        __syncthreads();
        if constexpr (FlushFn::active) {
            flush(i0, i1, part, W);
            if (FLUSH) __syncthreads();
            return;
        }
        for (int o = threadIdx.x; o < (i1 - i0) * NTT * 64; o += blockDim.x) {
            const int i = o / (NTT * 64), tt = (o / 64) % NTT, ll = o % 64;
            f4 sum = part[((i * W + 0) * NTT + tt) * 64 + ll];
            for (int w2 = 1; w2 < W; ++w2) sum += part[((i * W + w2) * NTT + tt) * 64 + ll];
            const int j = tt * 16 + ll % 16;
            const int64_t T = tmap(i0 + i);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = T * kTileR + 4 * (ll / 16) + r;
                if (j < M && row < rows) put(row, j, sum[r]);
            }
        }
        if (FLUSH) __syncthreads();   // (the next tiles write the same LDS)
    };
    if constexpr (NT > 0) {
        ready();
        // straight-line: tile i + DEPTH - 1's loads go to the slot tile i - 1 used, then tile i is computed
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            if (i + DEPTH - 1 < NT) load(i + DEPTH - 1, cw[(i + DEPTH - 1) % DEPTH], sw[(i + DEPTH - 1) % DEPTH]);
            tile(i, cw[i % DEPTH], sw[i % DEPTH]);
        }
    } else {
        // a ring of DEPTH tiles' loads: DEPTH - 1 in flight while one is computed. Everything loaded so far (the
        // activations, the first DEPTH - 1 tiles) is waited for here, once: the loop then starts from the state its
        // back edge has (DEPTH - 1 tiles in flight). Tile i + d is computed from slot d, its slot then refilled with
        // tile i + d + DEPTH ... by the load issued just before it (slot (d + DEPTH - 1) % DEPTH).
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0) (expcnt, lgkmcnt: no wait)
        ready();
        for (int i = 0; i < nt; i += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                if (i + d >= nt) break;
                load(i + d + DEPTH - 1, cw[(d + DEPTH - 1) % DEPTH], sw[(d + DEPTH - 1) % DEPTH]);
                tile(i + d, cw[d], sw[d]);
                if constexpr (FLUSH > 0) {   // every FLUSH tiles (and the last): their sums out, the LDS free again
                    const int done = i + d + 1;
                    if (done % FLUSH == 0 || done == nt) split_k_out(done - 1 - (done - 1) % FLUSH, done);
                }
            }
        }
    }
    if (MODE == kKeepParts) {
        __syncthreads();
        return;
    }
    if (MODE == kSplitK && FLUSH == 0) split_k_out(0, nt);
}

}  // namespace gv
