// sample.hip - the sampler and the two acceptance rules on the GPU (C2).
//
//   Sampler::sample       sampler.cpp:16-50        T <= 0: the first argmax. Else the candidates (top_k, else the
//                                                   top `cap` = 1024, ties to the lower index) by logit descending,
//                                                   e = exp((l - max) / T) in float, their sum in double, top-p the
//                                                   smallest prefix whose probability reaches p, r = kept x u, the
//                                                   first candidate where r - (e_0 + .. + e_i) <= 0.
//   sample-and-match      geode.cpp:318-374        each verified row sampled with its own uniform; a draft stands
//                                                   while the row before samples exactly it.
//   textbook rule         (Leviathan et al. 2023, Alg. 1; not in the reference) accept d ~ q with probability
//                                                   min(1, p(d) / q(d)); at the first rejection a token from
//                                                   max(0, p - q) by inverse CDF in index order; a bonus from p_k
//                                                   when every draft stands.
//
// Two paths. The candidate path (fast_*) decides a nucleus of top_p < 1, or the top-K candidates, among the elements
// at or above one logit: binned chunk summaries, the elements above the row's threshold bin collected grouped by bin,
// only the bins where the prefix ends and where the draw lands put in order (its comment below). A row it cannot
// decide goes to the walks, which decide any row:
//
// The sorted order of a row (logit descending, index ascending) is walked without sorting the row: a walk finds the
// element where the running weight of that order first reaches a target, by three histogram levels of an
// order-preserving 32-bit key (bits 31..21, 20..10, 9..0), each level a pass of S workgroups a row over the
// elements under the bits fixed so far. The last level leaves a key tau, the ties of it taken (in index order) and
// the weight of the elements before them; the pass that builds the last level's histogram also lists the few
// elements under its 22-bit prefix, from which the element itself and tie ranks are read. The weight is 1 a
// candidate for the top-K candidates, and e = exp((l - max) / T) for the full-vocabulary nucleus (its top-p prefix,
// then the draw within it): no candidate limit there. Each pass decides the previous level itself from that
// level's histogram (its loads in flight with the row's), so a level costs one launch.
//
// The top-K candidates (at most 16,384) are collected by the count walk's last pass and sorted in LDS by one
// workgroup a row, which then runs the reference's nucleus arithmetic on them as written. The histogram weights are
// summed by double atomics and the other double sums as parallel reductions: they differ from the reference's
// sequential sums in the last bits (~1e-15 relative), which moves a decision only when a uniform or top_p falls that
// close to a boundary; expf is the device's (within 1 ulp of glibc's).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <climits>
#include <cmath>
#include <vector>

#include "../../include/geode_verify.h"
#include "common.hpp"
#include "kernels.hpp"

namespace gv {
namespace {

constexpr int kPass = 256;        // threads of a row-pass workgroup
constexpr int kLoads = 16;        // values a thread holds in a pass
constexpr int kChunk = kPass * kLoads;   // values a row-pass workgroup takes at most
constexpr int kMaxChunks = 64;    // workgroups a row at most (a vocabulary up to 262,144)
constexpr int kMaxVocab = kMaxChunks * kChunk;   // the entry points refuse a larger vocabulary before any work
constexpr int kBins = 2048;       // bins of a histogram level (the last level uses 1024)
constexpr int kSortThreads = 1024;
constexpr int kMaxCand = 16384;   // top-K candidates a row can keep (the full-vocabulary nucleus has no limit)
constexpr int kList = 1024;       // elements a walk lists under its last level's prefix
constexpr int kSampleRows = 64;   // rows gv_sample_rows takes at most
constexpr int kFB = 48;        // the candidate path's bins of a chunk's summary (down to exp(-12) of its largest e)
constexpr int kFCap = 4096;    // elements a row collects at most on the candidate path

__host__ __device__ constexpr int level_shift(int l) { return l == 0 ? 21 : l == 1 ? 10 : 0; }
__host__ __device__ constexpr int level_bins(int l) { return l == 2 ? 1024 : 2048; }

// float -> a key whose unsigned order is the float order (-0 taken as +0: equal floats, equal keys)
__device__ inline uint32_t fkey(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float key_val(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

// e = exp((l - max) / T) as the reference computes it (float), sampler.cpp:31
__device__ inline float e_of(float l, float mx, float T) { return expf(__fdiv_rn(__fsub_rn(l, mx), T)); }

template <typename T>
__device__ inline T wave_incl_scan(T v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}

// exclusive scan over the workgroup (thread order); tot: the total; tmp: LDS of 16 T
template <typename T>
__device__ inline T block_excl_scan(T v, T *tmp, T &tot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const T incl = wave_incl_scan(v);
    __syncthreads();   // tmp may still be read by an earlier scan
    if (lane == 63) tmp[wave] = incl;
    __syncthreads();
    T base = 0, all = 0;
    for (int w = 0; w < nw; ++w) {
        if (w < wave) base += tmp[w];
        all += tmp[w];
    }
    tot = all;
    return base + incl - v;
}

template <typename T>
__device__ inline T block_sum(T v, T *tmp) {
    T tot;
    (void)block_excl_scan(v, tmp, tot);
    return tot;
}

// ---------------------------------------------------------------- the state of a row
struct LevelHist {   // a row's histogram of one level: element counts and weights per bin
    uint32_t cnt[kBins];
    double w[kBins];
};
enum { H_L1 = 0, H_L2P = 1, H_L3P = 2, H_L2D = 3, H_L3D = 4, kHists = 5 };

// A walk down the sorted order to the element where the running weight first reaches a target.
struct Walk {
    uint32_t prefix, mask;   // the key bits fixed so far
    double t;                // the weight still to reach among the elements under prefix (inf: to the last one)
    double above;            // the weight of the elements before them
    uint32_t above_cnt;      // their count
    uint32_t tau, n, c;      // at the end: the key reached, its ties taken (in index order), its ties there are
    double w_tau;            // a tie's weight
};

struct RowInfo {
    float mx;          // the row's largest logit
    int32_t pick;      // the sampled (or first largest) index
    double sum;        // the nucleus's denominator: the whole row's e (full vocabulary) or the candidates'
    double kept;       // e of the kept prefix
    uint32_t keep;     // its length
    uint32_t unused;
    // the walks' states, a slot a pass (a pass reads the previous pass's slot while its own workgroup 0 writes the
    // next): the top-p (top-K) walk after levels 0 and 1 and at its end, the draw's after levels 0 and 1 (its last
    // level is decided where the pick is read)
    Walk wk[5];
    __device__ const Walk &p() const { return wk[2]; }
};
enum { W_P0 = 0, W_P1 = 1, W_P = 2, W_D0 = 3, W_D1 = 4 };
enum { L_P = 0, L_D = 1 };          // the two walks' lists
enum { N_CAND = 0, N_LIST = 1 };    // a row's counters: candidates collected, elements listed (P, then D)

struct Rows {   // rows [0, R1) of x1, then rows of x2, ld floats apart; a row in S chunks of C values
    const float *x1, *x2;
    int64_t ld;
    int R1, V, S, C;
    __device__ const float *row(int r) const {
        return r < R1 ? x1 + static_cast<int64_t>(r) * ld : x2 + static_cast<int64_t>(r - R1) * ld;
    }
};

struct FRow {
    uint32_t n;        // elements collected (more than kFCap: the row is not decided here)
    int32_t ok;        // the row is decided here
    uint64_t last;     // the kept prefix's last element, (key << 32) | ~index: x is kept iff its own is at least this
    uint32_t top_key;  // the row's largest key
    int32_t jc;        // the last bin collected (from the top)
};

struct Ws {   // device arrays of R rows
    RowInfo *info;        // [R]
    uint32_t *pmax;       // [R][kMaxChunks] a chunk's largest key
    int32_t *pidx;        //                 the lowest index holding it
    double *psum;         //                 a chunk's e sum
    LevelHist *h;         // [R][kHists]
    uint32_t *cnt;        // [R][4] counters (N_*), zeroed by the first pass
    uint64_t *cand;       // [R][kMaxCand] (key << 32) | ~index
    uint64_t *lst;        // [R][2][kList] (key << 32) | index
    int32_t *picks;       // [R] the rows' picks
    double *u;            // [R] the uniforms
    struct FStat *fs;     // [R][kMaxChunks] the candidate path's chunk summaries
    struct FRow *fr;      // [R] its row states
    uint32_t *fbc;        // [R][kFB] its bins' collected elements
};

// ---------------------------------------------------------------- loads
__device__ inline void preload(const float *row, int c0, int c1, float (&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) v[u] = row[min(c0 + u * kPass + static_cast<int>(threadIdx.x), c1 - 1)];
}

// ---------------------------------------------------------------- a walk's steps (every thread of a workgroup)
struct WalkLds {
    double tmp_d[16];
    uint32_t tmp_u[16];
    uint32_t first, lastp1;
};

// Level `level` of the walk `in` from its histogram: the first nonempty bin (from the top) where the running weight
// reaches in.t, else (rounding left the target past the end) the last nonempty bin, whose elements are then all
// taken. The next state goes to `out` (LDS). Workgroups of 256 or 1024 threads.
__device__ void walk_level(const LevelHist &h, int level, const Walk in, Walk &out, WalkLds &L) {
    const int nb = level_bins(level), sh = level_shift(level), per = nb / static_cast<int>(blockDim.x);
    const int tid = threadIdx.x;
    double w[8];
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int b = nb - 1 - (tid * per + j);
        c[j] = j < per ? h.cnt[b] : 0u;
        w[j] = j < per ? h.w[b] : 0.0;
    }
    double lw = 0.0;
    uint32_t lc = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        lw += w[j];
        lc += c[j];
    }
    if (tid == 0) {
        L.first = UINT_MAX;
        L.lastp1 = 0;
    }
    double wtot;
    const double wex = block_excl_scan(lw, L.tmp_d, wtot);   // (its barriers publish the resets above)
    uint32_t ctot;
    const uint32_t cex = block_excl_scan(lc, L.tmp_u, ctot);
    double acc = wex;
    uint32_t first = UINT_MAX, lastp1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (j < per && c[j]) {
            if (first == UINT_MAX && acc + w[j] >= in.t) first = static_cast<uint32_t>(tid * per + j);
            lastp1 = static_cast<uint32_t>(tid * per + j + 1);
        }
        acc += w[j];
    }
    if (first != UINT_MAX) atomicMin(&L.first, first);
    if (lastp1) atomicMax(&L.lastp1, lastp1);
    __syncthreads();
    const bool reached = L.first != UINT_MAX;
    const uint32_t rank = reached ? L.first : L.lastp1 - 1;   // (a walk's elements are never none)
    if (tid == static_cast<int>(rank / per)) {
        const int j0 = static_cast<int>(rank % per);
        double above = wex;
        uint32_t cabove = cex, cj = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < j0) {
                above += w[j];
                cabove += c[j];
            }
            if (j == j0) cj = c[j];
        }
        const uint32_t bin = static_cast<uint32_t>(nb - 1) - rank;
        Walk s = in;
        s.above += above;
        s.above_cnt += cabove;
        s.t = reached ? in.t - above : INFINITY;
        s.prefix |= bin << sh;
        s.mask |= static_cast<uint32_t>(nb - 1) << sh;
        if (level == 2) {
            s.tau = s.prefix;
            s.c = cj;
        }
        out = s;
    }
    __syncthreads();
}

// after the last level (one thread): a tie's weight and the ties taken through the target
__device__ void walk_finish(Walk &s, bool mass, float mx, float T) {
    s.w_tau = mass ? static_cast<double>(e_of(key_val(s.tau), mx, T)) : 1.0;
    uint32_t n = s.c;
    if (!isinf(s.t)) {
        const double q = ceil(s.t / s.w_tau);
        n = q < 1.0 ? 1u : (q >= static_cast<double>(s.c) ? s.c : static_cast<uint32_t>(q));
        while (n < s.c && static_cast<double>(n) * s.w_tau < s.t) ++n;   // (the division's rounding)
    }
    s.n = n;
}

// ---------------------------------------------------------------- row passes: grid (S, R), kPass threads
// (a chunk is at most kChunk values: thread t holds the values c0 + t + 256 u, u < kLoads)
struct PassOut {
    LevelHist *g;
    double *chunk_e;     // every element's e summed (the mass walk's first level), or null
    uint64_t *list;      // the last level: the elements under the prefix listed, or null
    uint32_t *nlist;
    uint64_t *cand;      // the count walk's last level: the elements above the prefix collected, or null
    uint32_t *ncand;
};

struct PassLds {
    uint32_t lc[kBins];
    double lw[kBins];
    uint32_t tmp_u[16];
    double tmp_d[16];
    uint32_t base_l, base_c;
};

// A chunk's elements under the walk's prefix into level `level`'s histogram (LDS, then the row's by atomics);
// mass: weights e, else 1. The listed and collected elements get their slots in one reservation a workgroup.
template <bool MASS>
__device__ void hist_chunk(int c0, int c1, const float (&v)[kLoads], uint32_t prefix, uint32_t mask, int level,
                           float mx, float T, PassLds &S, const PassOut &o) {
    const int tid = threadIdx.x, nb = level_bins(level), sh = level_shift(level);
    for (int b = tid; b < nb; b += kPass) {
        S.lc[b] = 0;
        S.lw[b] = 0.0;
    }
    __syncthreads();
    double acc = 0.0;
    uint32_t nl = 0, nc = 0;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        if (c0 + u * kPass + tid >= c1) continue;
        const uint32_t k = fkey(v[u]);
        const bool under = (k & mask) == prefix;
        if (MASS && (o.chunk_e || under)) {
            const float e = e_of(v[u], mx, T);
            acc += static_cast<double>(e);
            if (under) atomicAdd(&S.lw[(k >> sh) & (nb - 1)], static_cast<double>(e));
        }
        if (under) atomicAdd(&S.lc[(k >> sh) & (nb - 1)], 1u);
        nl += under;
        nc += (k & mask) > prefix;
    }
    if (o.chunk_e) *o.chunk_e = acc;
    if (o.list || o.cand) {
        uint32_t tl, tc;
        uint32_t al = block_excl_scan(o.list ? nl : 0u, S.tmp_u, tl);
        uint32_t ac = block_excl_scan(o.cand ? nc : 0u, S.tmp_u, tc);
        if (tid == 0) {
            S.base_l = tl ? atomicAdd(o.nlist, tl) : 0u;
            S.base_c = tc ? atomicAdd(o.ncand, tc) : 0u;
        }
        __syncthreads();
        al += S.base_l;
        ac += S.base_c;
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int i = c0 + u * kPass + tid;
            if (i >= c1) continue;
            const uint32_t k = fkey(v[u]);
            if (o.list && (k & mask) == prefix) {
                if (al < static_cast<uint32_t>(kList)) o.list[al] = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(i);
                ++al;
            }
            if (o.cand && (k & mask) > prefix) {
                if (ac < static_cast<uint32_t>(kMaxCand))
                    o.cand[ac] = (static_cast<uint64_t>(k) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
                ++ac;
            }
        }
    }
    __syncthreads();
    for (int b = tid; b < nb; b += kPass)
        if (S.lc[b]) {
            atomicAdd(&o.g->cnt[b], S.lc[b]);
            atomicAdd(&o.g->w[b], MASS ? S.lw[b] : static_cast<double>(S.lc[b]));
        }
}

// pass 0: a chunk's largest key and the lowest index holding it; the row's histograms and counters zeroed for the
// passes after it (a share each workgroup)
template <bool ZERO>
__global__ __launch_bounds__(kPass) void max_pass(Rows rs, Ws ws) {
    __shared__ uint64_t red[kPass / 64];
    const int w = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    const float *row = rs.row(r);
    const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
    float v[kLoads];
    preload(row, c0, c1, v);
    if (ZERO) {
        uint32_t *h = reinterpret_cast<uint32_t *>(ws.h + r * kHists);
        constexpr int words = static_cast<int>(sizeof(LevelHist) * kHists / 4);
        for (int i = w * kPass + tid; i < words; i += rs.S * kPass) h[i] = 0u;
        if (w == 0 && tid < 4) ws.cnt[r * 4 + tid] = 0u;
    }
    uint64_t best = 0;   // (key << 32) | ~index: the largest is the largest key at the lowest index
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        const int i = c0 + u * kPass + tid;
        if (i < c1) best = max(best, (static_cast<uint64_t>(fkey(v[u])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i)));
    }
    for (int o = 32; o > 0; o >>= 1) best = max(best, static_cast<uint64_t>(__shfl_xor(best, o, 64)));
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kPass / 64; ++i) best = max(best, red[i]);
        ws.pmax[r * kMaxChunks + w] = static_cast<uint32_t>(best >> 32);
        ws.pidx[r * kMaxChunks + w] = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(best));
    }
}

// the first argmax of each row from its chunks' (a wave a row, a lane a chunk)
__global__ __launch_bounds__(64) void argmax_reduce(Ws ws, int S) {
    const int r = blockIdx.x, lane = threadIdx.x;
    uint64_t best = 0;
    if (lane < S)
        best = (static_cast<uint64_t>(ws.pmax[r * kMaxChunks + lane]) << 32) |
               (0xFFFFFFFFu - static_cast<uint32_t>(ws.pidx[r * kMaxChunks + lane]));
    for (int o = 32; o > 0; o >>= 1) best = max(best, static_cast<uint64_t>(__shfl_xor(best, o, 64)));
    if (lane == 0) {
        const int32_t pick = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(best));
        ws.info[r].pick = pick;
        ws.info[r].mx = key_val(static_cast<uint32_t>(best >> 32));
        ws.picks[r] = pick;
    }
}

// pass 1: the first level's histogram; mass: with the row's max and each chunk's e sum
template <bool MASS>
__global__ __launch_bounds__(kPass) void level1_pass(Rows rs, Ws ws, float T) {
    __shared__ PassLds S;
    const int w = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    const float *row = rs.row(r);
    const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
    float v[kLoads];
    preload(row, c0, c1, v);
    float mx = 0.0f;
    if (MASS) {   // the row's largest logit from its chunks'
        uint32_t mk = ws.pmax[r * kMaxChunks];
        for (int i = 1; i < rs.S; ++i) mk = max(mk, ws.pmax[r * kMaxChunks + i]);
        mx = key_val(mk);
        if (w == 0 && tid == 0) ws.info[r].mx = mx;
    }
    double part = 0.0;
    const PassOut o{ws.h + r * kHists + H_L1, MASS ? &part : nullptr, nullptr, nullptr, nullptr, nullptr};
    hist_chunk<MASS>(c0, c1, v, 0u, 0u, 0, mx, T, S, o);
    if (MASS) {
        const double s = block_sum(part, S.tmp_d);
        if (tid == 0) ws.psum[r * kMaxChunks + w] = s;
    }
}

enum Stage {
    ST_P1 = 0,   // start the top-p (top-K) walk: level 0 from the first histogram; level 1's histogram
    ST_P2 = 1,   // level 1; level 2's histogram, the elements under the prefix listed (and the top-K's above it)
    ST_D1 = 2,   // finish the top-p walk (the kept prefix), start the draw: level 0; level 1's histogram
    ST_D2 = 3    // level 1 of the draw; level 2's histogram, the elements under the prefix listed
};

// passes 2..5 of the walks (mass: the nucleus and the draw; count: the top-K walk, stages P1 and P2 only)
template <bool MASS, int STAGE>
__global__ __launch_bounds__(kPass) void walk_pass(Rows rs, Ws ws, float T, float top_p, int K) {
    __shared__ PassLds S;
    __shared__ Walk s, s2;
    __shared__ WalkLds L;
    const int w = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    RowInfo &info = ws.info[r];
    LevelHist *h = ws.h + r * kHists;
    const float *row = rs.row(r);
    const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
    float v[kLoads];
    preload(row, c0, c1, v);   // (in flight while the previous level is decided)
    const float mx = MASS ? info.mx : 0.0f;
    int level = 1, out = H_L2P;
    if (STAGE == ST_P1) {
        double target = static_cast<double>(K);
        if (MASS) {
            double tot = 0.0;   // the row's e sum, chunks in order
            for (int i = 0; i < rs.S; ++i) tot += ws.psum[r * kMaxChunks + i];
            target = top_p < 1.0f ? static_cast<double>(top_p) * tot : INFINITY;
            if (w == 0 && tid == 0) info.sum = tot;
        }
        walk_level(h[H_L1], 0, Walk{0u, 0u, target, 0.0, 0u, 0u, 0u, 0u, 0.0}, s, L);
    } else if (STAGE == ST_P2) {
        walk_level(h[H_L2P], 1, info.wk[W_P0], s, L);
        level = 2;
        out = H_L3P;
    } else if (STAGE == ST_D1) {
        walk_level(h[H_L3P], 2, info.wk[W_P1], s2, L);
        if (tid == 0) {
            walk_finish(s2, true, mx, T);
            const double kept = s2.above + static_cast<double>(s2.n) * s2.w_tau;
            if (w == 0) {
                info.wk[W_P] = s2;
                info.keep = s2.above_cnt + s2.n;
                info.kept = kept;
            }
            s2 = Walk{0u, 0u, kept * ws.u[r], 0.0, 0u, 0u, 0u, 0u, 0.0};
        }
        __syncthreads();
        walk_level(h[H_L1], 0, s2, s, L);
        out = H_L2D;
    } else {
        walk_level(h[H_L2D], 1, info.wk[W_D0], s, L);
        level = 2;
        out = H_L3D;
    }
    if (w == 0 && tid == 0) info.wk[STAGE == ST_P1 ? W_P0 : STAGE == ST_P2 ? W_P1 : STAGE == ST_D1 ? W_D0 : W_D1] = s;
    const int wl = STAGE == ST_D2 ? L_D : L_P;
    const bool last = level == 2;
    const PassOut o{h + out, nullptr, last ? ws.lst + (static_cast<int64_t>(r) * 2 + wl) * kList : nullptr,
                    ws.cnt + r * 4 + N_LIST + wl,
                    (!MASS && last) ? ws.cand + static_cast<int64_t>(r) * kMaxCand : nullptr, ws.cnt + r * 4 + N_CAND};
    hist_chunk<MASS>(c0, c1, v, s.prefix, s.mask, level, mx, T, S, o);
}

// ---------------------------------------------------------------- the element of a key, the rank of an index
struct FindLds {
    uint32_t tmp_u[16];
    int found;
};

// The n-th (1-based) smallest index among the row's elements of key `key`, from the walk's list when it holds every
// element under the walk's last prefix, else by a scan of the row in index order (every thread of the workgroup)
__device__ int nth_of_key(const Rows &rs, const Ws &ws, int r, int wl, uint32_t key, uint32_t n, FindLds &F) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t m = ws.cnt[r * 4 + N_LIST + wl];
    if (tid == 0) F.found = -1;
    __syncthreads();
    if (m <= static_cast<uint32_t>(kList)) {
        const uint64_t *lst = ws.lst + (static_cast<int64_t>(r) * 2 + wl) * kList;
        for (uint32_t j = tid; j < m; j += nthr) {
            const uint64_t e = lst[j];
            if (static_cast<uint32_t>(e >> 32) != key) continue;
            const uint32_t x = static_cast<uint32_t>(e);
            uint32_t below = 0;
            for (uint32_t q = 0; q < m; ++q) {
                const uint64_t f = lst[q];
                below += static_cast<uint32_t>(f >> 32) == key && static_cast<uint32_t>(f) < x;
            }
            if (below + 1 == n) F.found = static_cast<int>(x);
        }
        __syncthreads();
        return F.found;
    }
    // (more elements under the prefix than a list holds: a scan, each thread a run of consecutive indices)
    const float *row = rs.row(r);
    uint32_t carry = 0;
    for (int b0 = 0; b0 < rs.V; b0 += nthr * kLoads) {
        const int x0 = b0 + tid * kLoads, x1 = min(rs.V, x0 + kLoads);
        uint32_t mine = 0;
        for (int x = x0; x < x1; ++x) mine += fkey(row[x]) == key;
        uint32_t tot;
        uint32_t at = carry + block_excl_scan(mine, F.tmp_u, tot);
        if (at < n && at + mine >= n)
            for (int x = x0; x < x1; ++x)
                if (fkey(row[x]) == key && ++at == n) F.found = x;
        carry += tot;
        if (carry >= n) break;
    }
    __syncthreads();
    return F.found;
}

// how many of the row's elements of key `key` have an index below x (the same two ways)
__device__ uint32_t rank_of_key(const Rows &rs, const Ws &ws, int r, int wl, uint32_t key, int x, FindLds &F) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t m = ws.cnt[r * 4 + N_LIST + wl];
    uint32_t below = 0;
    if (m <= static_cast<uint32_t>(kList)) {
        const uint64_t *lst = ws.lst + (static_cast<int64_t>(r) * 2 + wl) * kList;
        for (uint32_t j = tid; j < m; j += nthr) {
            const uint64_t e = lst[j];
            below += static_cast<uint32_t>(e >> 32) == key && static_cast<uint32_t>(e) < static_cast<uint32_t>(x);
        }
    } else {
        const float *row = rs.row(r);
        for (int i = tid; i < x; i += nthr) below += fkey(row[i]) == key;
    }
    return block_sum(below, F.tmp_u);
}

// whether index x (key kx) of row r is in its kept prefix: above the top-p walk's key, or one of its first n ties
__device__ bool in_kept(const Rows &rs, const Ws &ws, int r, int x, uint32_t kx, FindLds &F) {
    const Walk &p = ws.info[r].p();
    if (kx != p.tau) return kx > p.tau;
    if (p.n == p.c) return true;
    return rank_of_key(rs, ws, r, L_P, p.tau, x, F) < p.n;
}

// the draws of the full-vocabulary nuclei (a workgroup a row): the draw's last level, at most to the kept prefix's
// last element, the element from the lists
__global__ __launch_bounds__(kPass) void draw_pick(Rows rs, Ws ws, float T) {
    __shared__ Walk s;
    __shared__ WalkLds L;
    __shared__ FindLds F;
    const int r = blockIdx.x, tid = threadIdx.x;
    RowInfo &info = ws.info[r];
    walk_level(ws.h[r * kHists + H_L3D], 2, info.wk[W_D1], s, L);
    if (tid == 0) walk_finish(s, true, info.mx, T);
    __syncthreads();
    const Walk &p = info.p();
    const bool past = s.tau < p.tau || (s.tau == p.tau && s.n > p.n);   // rounding past the kept prefix: its last
    const int at = past ? nth_of_key(rs, ws, r, L_P, p.tau, p.n, F) : nth_of_key(rs, ws, r, L_D, s.tau, s.n, F);
    if (tid == 0) {
        const int pick = min(max(at, 0), rs.V - 1);   // (always found: the counts and the elements agree)
        info.pick = pick;
        ws.picks[r] = pick;
    }
}

// ---------------------------------------------------------------- the top-K candidates (count walk)
// A workgroup a row: the count walk's last level (tau, the ties taken); the candidates: those collected above the
// walk's last prefix, those under it above tau and the first ties of tau in index order; sorted by value descending,
// index ascending, in LDS; then the reference's nucleus on them as written (sampler.cpp:31-49): e_i = exp((l_i -
// max) / T), their sum, keep = the top-p prefix, kept = e_0 + .. + e_{keep-1}, and the draw of u[row]: the first
// i < keep where kept u <= e_0 + .. + e_i (else keep - 1).
template <int KP>
__global__ __launch_bounds__(kSortThreads) void cand_nucleus(Rows rs, Ws ws, float T, float top_p) {
    extern __shared__ uint64_t comp[];   // [KP]
    __shared__ Walk s;
    __shared__ WalkLds L;
    __shared__ uint32_t tmp_u[16];
    __shared__ double tmp_d[16];
    __shared__ int s_first;
    const int r = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x;
    RowInfo &info = ws.info[r];
    walk_level(ws.h[r * kHists + H_L3P], 2, info.wk[W_P1], s, L);
    if (tid == 0) {
        walk_finish(s, false, 0.0f, 1.0f);
        info.wk[W_P] = s;
    }
    __syncthreads();
    const int K = min(static_cast<int>(s.above_cnt + s.n), KP);
    const int above = static_cast<int>(min(ws.cnt[r * 4 + N_CAND], static_cast<uint32_t>(K)));
    const uint64_t *cand = ws.cand + static_cast<int64_t>(r) * kMaxCand;
    for (int i = tid; i < KP; i += nthr) comp[i] = i < above ? cand[i] : 0ull;
    __syncthreads();
    // the prefix's elements above tau, then the first n ties of tau (in index order), after the collected ones
    const uint32_t m = ws.cnt[r * 4 + N_LIST + L_P];
    const uint32_t tau = s.tau, n = s.n;
    if (m <= static_cast<uint32_t>(kList)) {
        const uint64_t *lst = ws.lst + static_cast<int64_t>(r) * 2 * kList;
        uint32_t carry = 0;
        for (uint32_t j0 = 0; j0 < m; j0 += nthr) {   // those above tau: any order
            const uint32_t j = j0 + tid;
            const uint64_t e = j < m ? lst[j] : 0ull;
            const uint32_t f = j < m && static_cast<uint32_t>(e >> 32) > tau;
            uint32_t tot;
            const uint32_t at = carry + block_excl_scan(f, tmp_u, tot);
            if (f && above + static_cast<int>(at) < K)
                comp[above + at] = (e & 0xFFFFFFFF00000000ull) | (0xFFFFFFFFu - static_cast<uint32_t>(e));
            carry += tot;
        }
        const int base = above + static_cast<int>(carry);
        for (uint32_t j = tid; j < m; j += nthr) {   // the ties: by their rank in index order
            const uint64_t e = lst[j];
            if (static_cast<uint32_t>(e >> 32) != tau) continue;
            uint32_t below = 0;
            for (uint32_t q = 0; q < m; ++q)
                below += static_cast<uint32_t>(lst[q] >> 32) == tau && static_cast<uint32_t>(lst[q]) < static_cast<uint32_t>(e);
            if (below < n && base + static_cast<int>(below) < K)
                comp[base + below] = (e & 0xFFFFFFFF00000000ull) | (0xFFFFFFFFu - static_cast<uint32_t>(e));
        }
    } else {   // (more elements under the prefix than the list holds: a scan of the row in index order)
        const float *row = rs.row(r);
        const uint32_t pmask = s.mask & ~1023u, pre22 = s.prefix & ~1023u;
        uint32_t ca = 0, ct = 0;
        for (int b0 = 0; b0 < rs.V; b0 += nthr * kLoads) {
            const int x0 = b0 + tid * kLoads, x1 = min(rs.V, x0 + kLoads);
            uint32_t na = 0, nt = 0;
            for (int x = x0; x < x1; ++x) {
                const uint32_t k = fkey(row[x]);
                na += (k & pmask) == pre22 && k > tau;
                nt += k == tau;
            }
            uint32_t ta, tt;
            uint32_t aa = ca + block_excl_scan(na, tmp_u, ta);
            uint32_t at = ct + block_excl_scan(nt, tmp_u, tt);
            for (int x = x0; x < x1; ++x) {
                const uint32_t k = fkey(row[x]);
                const uint64_t e = (static_cast<uint64_t>(k) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(x));
                if ((k & pmask) == pre22 && k > tau) {
                    if (above + static_cast<int>(aa) < K) comp[above + aa] = e;
                    ++aa;
                }
                if (k == tau) {
                    if (at < n && K - static_cast<int>(n) + static_cast<int>(at) >= 0) comp[K - static_cast<int>(n) + at] = e;
                    ++at;
                }
            }
            ca += ta;
            ct += tt;
        }
    }
    __syncthreads();
    // bitonic sort, descending. Pair i of a stage of stride s <= 64 has both elements in [128 (i / 64), + 128): a
    // wave's 64 consecutive pairs keep the same 128 elements from one such stage to the next, so between two of them
    // the wave only waits for its own LDS writes; a workgroup barrier follows every other stage.
    for (int size = 2; size <= KP; size <<= 1)
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int i = tid; i < KP / 2; i += nthr) {
                const int lo = 2 * stride * (i / stride) + (i % stride), hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t a = comp[lo], b = comp[hi];
                if ((a < b) == desc) {
                    comp[lo] = b;
                    comp[hi] = a;
                }
            }
            const int next = stride > 1 ? stride / 2 : size;   // the next stage's stride (size * 2 / 2)
            if (stride <= 64 && next <= 64 && !(stride == 1 && size == KP)) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else {
                __syncthreads();
            }
        }
    const float mx = key_val(static_cast<uint32_t>(comp[0] >> 32));
    auto e_at = [&](int i) { return e_of(key_val(static_cast<uint32_t>(comp[i] >> 32)), mx, T); };
    double part = 0.0;
    for (int i = tid; i < K; i += nthr) part += static_cast<double>(e_at(i));
    const double sum = block_sum(part, tmp_d);
    int keep = K;
    if (top_p < 1.0f) {   // the first i where acc += e_i / sum reaches top_p
        if (tid == 0) s_first = K;
        double carry = 0.0;
        for (int c0 = 0; c0 < K; c0 += nthr) {
            const int i = c0 + tid;
            const double t = i < K ? static_cast<double>(e_at(i)) / sum : 0.0;
            double tot;
            const double acc = carry + block_excl_scan(t, tmp_d, tot) + t;
            if (i < K && acc >= static_cast<double>(top_p)) atomicMin(&s_first, i);
            carry += tot;
            __syncthreads();
            if (s_first < K) break;
        }
        keep = s_first < K ? s_first + 1 : K;
    }
    __syncthreads();   // every thread has read s_first
    if (tid == 0) s_first = INT32_MAX;
    double kept = 0.0;
    for (int c0 = 0; c0 < keep; c0 += nthr) {
        const int i = c0 + tid;
        kept += block_sum(i < keep ? static_cast<double>(e_at(i)) : 0.0, tmp_d);
    }
    const double rr = kept * ws.u[r];
    double carry = 0.0;
    for (int c0 = 0; c0 < keep; c0 += nthr) {
        const int i = c0 + tid;
        const double t = i < keep ? static_cast<double>(e_at(i)) : 0.0;
        double tot;
        const double acc = carry + block_excl_scan(t, tmp_d, tot) + t;
        if (i < keep && rr - acc <= 0.0) atomicMin(&s_first, i);
        carry += tot;
        __syncthreads();
        if (s_first != INT32_MAX) break;
    }
    __syncthreads();
    if (tid == 0) {
        const int at = s_first != INT32_MAX ? s_first : keep - 1;   // rounding past the end: the last kept
        const int32_t pick = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(comp[at]));
        info.mx = mx;
        info.sum = sum;
        info.keep = static_cast<uint32_t>(keep);
        info.kept = kept;
        info.pick = pick;
        ws.picks[r] = pick;
    }
}

// ---------------------------------------------------------------- acceptance
// A call's results written into pinned host memory, then its sequence number `seq` to *done (null: none): the host
// polls that word instead of waiting for the stream. The calling thread's result stores come first in program order,
// and the system-scope fence makes them visible before the word; a workgroup whose other threads stored results
// fences in each of them and meets at a barrier first.
__device__ inline void post_seq(uint32_t *done, uint32_t seq) {
    if (!done) return;
    __threadfence_system();
    __hip_atomic_store(done, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// sample-and-match over the sampled rows (geode.cpp:331-350): out = the stood drafts then the first sampled token
// that is no draft; a draft stands only if it is no stop token either (stop[0..n_stop)); res = {emitted, kept}, then
// seq to *done (post_seq). fr (the candidate path's rows, or null): a row it did not decide gives res = {0, 0}.
template <typename BatchAt, typename StopAt>
__device__ inline void match_body(const int32_t *__restrict__ picks, BatchAt batch_at, int n, StopAt stop_at,
                                  int n_stop, int32_t *__restrict__ out, int *__restrict__ res,
                                  const FRow *__restrict__ fr, uint32_t *done, uint32_t seq) {
    __shared__ int32_t pick[32], next[32];
    __shared__ int stopped[32];
    const int t = threadIdx.x;
    if (fr && __ballot(t < n && fr[min(t, n - 1)].ok == 0)) {
        if (t == 0) {
            res[0] = 0;
            res[1] = 0;
            post_seq(done, seq);
        }
        return;
    }
    if (t < n) {
        pick[t] = picks[t];
        next[t] = t + 1 < n ? batch_at(t + 1) : -1;
        stopped[t] = 0;
    }
    __syncthreads();
    for (int j = t; j < n_stop; j += blockDim.x) {   // which rows sampled a stop token
        const int32_t sj = stop_at(j);
        for (int i = 0; i < n; ++i)
            if (sj == pick[i]) stopped[i] = 1;
    }
    __syncthreads();
    if (t != 0) return;
    int emitted = 0, kept = 1;
    for (int i = 0; i < n; ++i) {
        out[emitted++] = pick[i];
        if (i + 1 < n && pick[i] == next[i] && !stopped[i]) {
            ++kept;
            continue;
        }
        break;
    }
    res[0] = emitted;
    res[1] = kept;
    post_seq(done, seq);
}

__global__ __launch_bounds__(64) void match_kernel(const int32_t *__restrict__ picks, const int32_t *__restrict__ batch,
                                                   int n, const int32_t *__restrict__ stop, int n_stop,
                                                   int32_t *__restrict__ out, int *__restrict__ res,
                                                   const FRow *__restrict__ fr) {
    match_body(picks, [&](int i) { return batch[i]; }, n, [&](int j) { return stop[j]; }, n_stop, out, res, fr, nullptr,
               0u);
}

// the same with the batch and up to 32 stop tokens as kernel arguments (no input copy)
struct MatchIn {
    int32_t batch[32];
    int32_t stop[32];
};

// greedy (T <= 0): each row's first argmax from its chunks' maxima (max_pass), then the decisions; one wave
__global__ __launch_bounds__(64) void greedy_match_kernel(Ws ws, int S, MatchIn in, int n, int n_stop,
                                                          int32_t *__restrict__ out, int *__restrict__ res,
                                                          uint32_t *done, uint32_t seq) {
    __shared__ int32_t pk[32];
    __shared__ uint64_t cm[32 * kMaxChunks];
    const int lane = threadIdx.x;
    for (int i = lane; i < n * S; i += 64) {   // (every row's chunk maxima, their loads independent)
        const int r = i / S, c = i - r * S;
        cm[r * kMaxChunks + c] = (static_cast<uint64_t>(ws.pmax[r * kMaxChunks + c]) << 32) |
                                 (0xFFFFFFFFu - static_cast<uint32_t>(ws.pidx[r * kMaxChunks + c]));
    }
    __syncthreads();
    for (int r = 0; r < n; ++r) {
        uint64_t b = lane < S ? cm[r * kMaxChunks + lane] : 0ull;
        for (int o = 32; o > 0; o >>= 1) b = max(b, static_cast<uint64_t>(__shfl_xor(b, o, 64)));
        if (lane == 0) pk[r] = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(b));
    }
    __syncthreads();
    match_body(pk, [&](int i) { return in.batch[i]; }, n, [&](int j) { return in.stop[j]; }, n_stop, out, res,
               static_cast<const FRow *>(nullptr), done, seq);
}
__global__ __launch_bounds__(64) void match_args_kernel(const int32_t *__restrict__ picks, MatchIn in, int n,
                                                        int n_stop, int32_t *__restrict__ out, int *__restrict__ res,
                                                        const FRow *__restrict__ fr, uint32_t *done, uint32_t seq) {
    match_body(picks, [&](int i) { return in.batch[i]; }, n, [&](int j) { return in.stop[j]; }, n_stop, out, res,
               fr, done, seq);
}

// The presence penalty of the generate loop (geode.cpp:236-255) on the verified rows, in place: row i (a workgroup)
// loses `penalty` at each of the answer's seen tokens (distinct) and at each draft batch[j], 1 <= j <= i, that is
// new (fresh[j]: in neither `seen` nor an earlier draft), the tokens rows 0..i-1 sampled if their drafts stood (a
// row after a fallen draft is never used). One subtraction a token, as the reference's once-each list.
__global__ void penalty_kernel(float *__restrict__ logits, int64_t ld, const int32_t *__restrict__ seen, int n_seen,
                               const int32_t *__restrict__ batch, const int32_t *__restrict__ fresh, float penalty) {
    float *lg = logits + static_cast<int64_t>(blockIdx.x) * ld;
    for (int j = threadIdx.x; j < n_seen; j += blockDim.x) lg[seen[j]] -= penalty;
    for (int j = 1 + static_cast<int>(threadIdx.x); j <= static_cast<int>(blockIdx.x); j += blockDim.x)
        if (fresh[j]) lg[batch[j]] -= penalty;
}

// max(0, p_x - q_x) of a row pair (target row rp, draft row rq): p_x = e_x / kept over the target's kept prefix (0
// outside it), q_x likewise
struct Residual {
    const float *tp, *tq;
    float mxp, mxq, T;
    double keptp, keptq;
    Walk P, Q;
    int rp, rq;
    // (every thread) the residual of the elements x0 + j, j < kLoads, below c1, into v; the partly taken ties of the
    // walks' keys ranked through the lists
    __device__ void run(const Rows &rs, const Ws &ws, int x0, int c1, double (&v)[kLoads], FindLds &F,
                        int *s_flag) const {
        float lp[kLoads], lq[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {   // (the loads first, all in flight)
            const int x = min(x0 + j, c1 - 1);
            lp[j] = tp[x];
            lq[j] = tq[x];
        }
        bool tied = false;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            v[j] = 0.0;
            if (x0 + j >= c1) continue;
            const uint32_t kp = fkey(lp[j]), kq = fkey(lq[j]);
            const bool inp = kp > P.tau || (kp == P.tau && P.n == P.c);
            const bool inq = kq > Q.tau || (kq == Q.tau && Q.n == Q.c);
            tied |= (kp == P.tau && P.n < P.c) || (kq == Q.tau && Q.n < Q.c);
            const double p = inp ? static_cast<double>(e_of(lp[j], mxp, T)) / keptp : 0.0;
            const double q = inq ? static_cast<double>(e_of(lq[j], mxq, T)) / keptq : 0.0;
            v[j] = fmax(0.0, p - q);
        }
        // partly taken ties (rare): ranked one element at a time, the whole workgroup together
        if (threadIdx.x == 0) *s_flag = 0;
        __syncthreads();
        if (tied) *s_flag = 1;
        __syncthreads();
        if (!*s_flag) return;
        for (int t = 0; t < static_cast<int>(blockDim.x); ++t) {
            __syncthreads();
            if (static_cast<int>(threadIdx.x) == t) *s_flag = tied ? x0 : -1;
            __syncthreads();
            const int y0 = *s_flag;
            if (y0 < 0) continue;
            for (int j = 0; j < kLoads && y0 + j < c1; ++j) {
                const float a = tp[y0 + j], b = tq[y0 + j];
                const uint32_t kp = fkey(a), kq = fkey(b);
                const bool tp_ = kp == P.tau && P.n < P.c, tq_ = kq == Q.tau && Q.n < Q.c;
                if (!tp_ && !tq_) continue;
                const bool inp = tp_ ? rank_of_key(rs, ws, rp, L_P, P.tau, y0 + j, F) < P.n
                                     : (kp > P.tau || (kp == P.tau && P.n == P.c));
                const bool inq = tq_ ? rank_of_key(rs, ws, rq, L_P, Q.tau, y0 + j, F) < Q.n
                                     : (kq > Q.tau || (kq == Q.tau && Q.n == Q.c));
                if (static_cast<int>(threadIdx.x) == t) {
                    const double p = inp ? static_cast<double>(e_of(a, mxp, T)) / keptp : 0.0;
                    const double q = inq ? static_cast<double>(e_of(b, mxq, T)) / keptq : 0.0;
                    v[j] = fmax(0.0, p - q);
                }
            }
        }
        __syncthreads();
    }
};

// The textbook rule (target rows 0..k, draft rows k+1..2k, their nuclei and draws done; grid S, or 1 when greedy).
// Every workgroup takes the decisions: d_i stands with probability min(1, p_i(d_i) / q_i(d_i)); at the first
// rejection, each workgroup sums the residual over its chunk, and the last to finish draws by inverse CDF in index
// order (u_res x the total; no residual mass: the target row's own draw). out: the stood drafts, then that token
// or, when all stand, the bonus (target row k's draw; its argmax when greedy). st[0] = emitted.
__global__ __launch_bounds__(kPass) void textbook_finish(Rows rs, Ws ws, int k, int greedy, float T,
                                                         const float *__restrict__ u_acc, float u_res,
                                                         double *__restrict__ rsum, uint32_t *__restrict__ done,
                                                         int32_t *__restrict__ out, int *__restrict__ st) {
    __shared__ FindLds F;
    __shared__ double tmp_d[16];
    __shared__ int s_last, s_w, s_first, s_lastpos, s_flag;
    __shared__ double s_goal;
    const int w = blockIdx.x, tid = threadIdx.x;
    int emitted = 0, rej = -1;
    bool fell = false;
    for (int i = 0; i < k; ++i) {
        const int d = min(max(ws.picks[k + 1 + i], 0), rs.V - 1);
        if (greedy) {   // the first argmaxes: the target's token is emitted; a different draft ends the step
            ++emitted;
            if (ws.picks[i] != d) {
                fell = true;
                break;
            }
            continue;
        }
        const RowInfo &P = ws.info[i], &Q = ws.info[k + 1 + i];
        const float lq = rs.row(k + 1 + i)[d], lp = rs.row(i)[d];
        const double qd = static_cast<double>(e_of(lq, Q.mx, T)) / Q.kept;
        const bool in_p = in_kept(rs, ws, i, d, fkey(lp), F);
        const double pd = in_p ? static_cast<double>(e_of(lp, P.mx, T)) / P.kept : 0.0;
        if (static_cast<double>(u_acc[i]) * qd < pd) {   // accepted with probability min(1, p/q)
            ++emitted;
            continue;
        }
        rej = i;
        break;
    }
    auto write_head = [&](int n_head) {   // the stood drafts (greedy: the target's argmaxes)
        for (int i = tid; i < n_head; i += kPass) out[i] = greedy ? ws.picks[i] : ws.picks[k + 1 + i];
    };
    if (rej < 0) {
        if (w == 0) {
            write_head(emitted);
            if (!fell) {   // every draft stood: the bonus
                if (tid == 0) out[emitted] = ws.picks[k];
                ++emitted;
            }
            if (tid == 0) st[0] = emitted;
        }
        return;
    }
    // the residual of pair rej over this chunk, thread tid taking a run of consecutive indices
    const RowInfo &P = ws.info[rej], &Q = ws.info[k + 1 + rej];
    const Residual R{rs.row(rej), rs.row(k + 1 + rej), P.mx, Q.mx, T, P.kept, Q.kept, P.p(), Q.p(), rej, k + 1 + rej};
    {
        double v[kLoads];
        const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
        R.run(rs, ws, c0 + tid * kLoads, c1, v, F, &s_flag);
        double acc = 0.0;
        for (int j = 0; j < kLoads; ++j) acc += v[j];
        const double s = block_sum(acc, tmp_d);
        if (tid == 0) {
            rsum[w] = s;
            __threadfence();
            s_last = atomicAdd(done, 1u) == static_cast<uint32_t>(gridDim.x - 1);
        }
        __syncthreads();
        if (!s_last) return;
        __threadfence();
    }
    // the last workgroup: the chunk where u_res x total is reached, then the element in it
    if (tid == 0) {
        double total = 0.0;
        for (int c = 0; c < rs.S; ++c) total += __hip_atomic_load(rsum + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_w = -1;
        if (total > 0.0) {
            const double goal = static_cast<double>(u_res) * total;
            double cum = 0.0;
            int last = -1;
            for (int c = 0; c < rs.S; ++c) {
                const double rc = __hip_atomic_load(rsum + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (rc > 0.0) last = c;
                if (rc > 0.0 && cum + rc >= goal) {
                    s_w = c;
                    break;
                }
                cum += rc;
            }
            // rounding left the goal past the end: the last chunk with mass, to its last positive weight
            s_goal = s_w < 0 ? INFINITY : goal - cum;
            if (s_w < 0) s_w = last;
        }
        s_first = INT32_MAX;
        s_lastpos = -1;
    }
    __syncthreads();
    int pick;
    if (s_w < 0) {
        pick = ws.picks[rej];   // no residual mass: the target row's own draw
    } else {
        double v[kLoads];
        const int c0 = s_w * rs.C, c1 = min(rs.V, c0 + rs.C), x0 = c0 + tid * kLoads;
        R.run(rs, ws, x0, c1, v, F, &s_flag);
        double mine = 0.0;
        for (int j = 0; j < kLoads; ++j) mine += v[j];
        double tot;
        double acc = block_excl_scan(mine, tmp_d, tot);
        const double goal = s_goal;
        for (int j = 0; j < kLoads; ++j) {
            if (!(v[j] > 0.0)) continue;
            acc += v[j];
            atomicMax(&s_lastpos, x0 + j);
            if (acc >= goal) {
                atomicMin(&s_first, x0 + j);
                break;
            }
        }
        __syncthreads();
        pick = s_first != INT32_MAX ? s_first : s_lastpos;   // rounding past the end: the last positive weight
    }
    write_head(emitted);
    if (tid == 0) {
        out[emitted] = pick;
        st[0] = emitted + 1;
    }
}

// ---------------------------------------------------------------- the candidate path (a nucleus of top_p < 1)
// The walks above go to any depth of the sorted order. A nucleus of top_p < 1 ends where its mass reaches top_p:
// with logits spread like a language model's (and C2's N(0, 3) at T 0.7) that is a few to a few thousand elements,
// all at or above one logit. The candidate path finds such a logit from a binned summary of each chunk, collects
// the elements at or above it (at most kFCap a row), sorts them in LDS and runs the reference's nucleus on them as
// written, then checks that the kept prefix ended inside them; a row it cannot decide (more elements, a prefix
// past them, a row whose largest value is not finite) is marked, and the caller takes the walks instead. Four
// launches instead of eight, none with histogram atomics:
//   fast_stats     a chunk's largest value m and its elements' counts and e-mass exp((l - m) / T) in bins of
//                  floor(4 l / T) (an e ratio of exp(1/4) a bin), the kFB bins from the chunk's top bin down;
//   fast_collect   the row's bins merged (a chunk's mass rescaled by exp((m - max) / T): an estimate), the first bin
//                  from the top where the mass reaches top_p (a 1e-3 margin and one bin more) or the count reaches
//                  K, the elements at or above it collected; every element's exact e summed a chunk, as the walks'
//                  first pass does;
//   fast_nucleus   a workgroup a row: the collected elements sorted (logit descending, index ascending), the
//                  nucleus, its draw, and the kept prefix written back in order;
//   fast_textbook  the textbook rule's decisions, and at a rejection the residual max(0, p - q) over the target's
//                  kept prefix (p is 0 elsewhere) in index order.
// A bin is a logit threshold (floor(4 l / T) does not decrease as l grows), so the collected elements are a top
// part of the sorted order and equal logits are collected together.

struct FStat {   // a chunk's summary
    uint32_t key;      // its largest key
    int32_t top;       // that value's bin
    float mass;        // its elements' exp((l - m) / T), m its largest value
    uint32_t unused;
    uint32_t cnt[kFB];   // elements a bin, bin top - j at j
    float w[kFB];        // their exp((l - m) / T)
};


struct FastU {   // kernel arguments: a uniform a row, the acceptance uniforms, the residual's
    double u[64];
    float acc[32];
    float res;
};

__device__ inline int fbin(float l, float s) { return static_cast<int>(fminf(fmaxf(floorf(l * s), -1.0e9f), 1.0e9f)); }
__device__ inline uint64_t comp_of(float l, uint32_t x) {
    return (static_cast<uint64_t>(fkey(l)) << 32) | (0xFFFFFFFFu - x);
}
__device__ inline uint32_t comp_index(uint64_t c) { return 0xFFFFFFFFu - static_cast<uint32_t>(c); }

// a[0, P) sorted descending (P a power of two; every thread of the workgroup, which holds whole waves). Pair i of a
// stage of stride s <= 64 has both elements in [128 (i / 64), + 128): a wave's 64 consecutive pairs keep the same
// 128 elements from one such stage to the next, so between two of them the wave only waits for its own LDS writes;
// a workgroup barrier follows every other stage, and the last.
__device__ void bitonic_desc(uint64_t *a, int P) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    for (int size = 2; size <= P; size <<= 1)
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int i = tid; i < P / 2; i += nthr) {
                const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1)), hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t x = a[lo], y = a[hi];
                if ((x < y) == desc) {
                    a[lo] = y;
                    a[hi] = x;
                }
            }
            const int next = stride > 1 ? stride / 2 : size;
            if (stride <= 64 && next <= 64 && !(stride == 1 && size == P)) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else {
                __syncthreads();
            }
        }
}

// one LDS atomic a wave: the lowest (highest) pos among the lanes where hit holds, pos rising with the lane
__device__ inline void wave_min_hit(bool hit, int pos, int *dst) {
    const uint64_t b = __ballot(hit);
    if (b && (threadIdx.x & 63) == __builtin_ctzll(b)) atomicMin(dst, pos);
}
__device__ inline void wave_max_hit(bool hit, int pos, int *dst) {
    const uint64_t b = __ballot(hit);
    if (b && (threadIdx.x & 63) == 63 - __builtin_clzll(b)) atomicMax(dst, pos);
}

// grid (S, R), kPass threads
__global__ __launch_bounds__(kPass) void fast_stats(Rows rs, Ws ws, float T) {
    __shared__ uint32_t scnt[kFB];
    __shared__ float sw[kFB];
    __shared__ uint64_t red[kPass / 64];
    __shared__ float redm[kPass / 64];
    const int w = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const float *row = rs.row(r);
    const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
    float v[kLoads];
    preload(row, c0, c1, v);
    if (tid < kFB) {
        scnt[tid] = 0u;
        sw[tid] = 0.0f;
    }
    uint64_t best = 0;
#pragma unroll
    for (int u = 0; u < kLoads; ++u)
        if (c0 + u * kPass + tid < c1) best = max(best, comp_of(v[u], static_cast<uint32_t>(c0 + u * kPass + tid)));
    for (int o = 32; o > 0; o >>= 1) best = max(best, static_cast<uint64_t>(__shfl_xor(best, o, 64)));
    if (lane == 0) red[tid >> 6] = best;
    __syncthreads();   // (also publishes the zeroed bins)
    best = max(max(red[0], red[1]), max(red[2], red[3]));
    const float mc = key_val(static_cast<uint32_t>(best >> 32)), s4 = 4.0f / T;
    const int top = fbin(mc, s4);
    float mass = 0.0f;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        if (c0 + u * kPass + tid >= c1) continue;
        const float e = e_of(v[u], mc, T);
        mass += e;
        const int b = top - fbin(v[u], s4);   // (>= 0 unless a value is NaN)
        if (static_cast<unsigned>(b) < static_cast<unsigned>(kFB)) {
            atomicAdd(&scnt[b], 1u);
            atomicAdd(&sw[b], e);
        }
    }
    for (int o = 32; o > 0; o >>= 1) mass += __shfl_xor(mass, o, 64);
    if (lane == 0) redm[tid >> 6] = mass;
    __syncthreads();
    FStat &o = ws.fs[r * kMaxChunks + w];
    if (tid < kFB) {
        o.cnt[tid] = scnt[tid];
        o.w[tid] = sw[tid];
    }
    if (tid == 0) {
        o.key = static_cast<uint32_t>(best >> 32);
        o.top = top;
        o.mass = (redm[0] + redm[1]) + (redm[2] + redm[3]);
    }
}

// grid (S, R), kPass threads. MASS: the full-vocabulary nucleus (top_p < 1); else the top-K candidates.
template <bool MASS>
__global__ __launch_bounds__(kPass) void fast_collect(Rows rs, Ws ws, float T, float top_p, int K) {
    __shared__ float sscale[kMaxChunks];
    __shared__ int soff[kMaxChunks];
    __shared__ uint32_t sq_c[4][64], sq_b[4][64];
    __shared__ double sq_w[4][64];
    __shared__ uint32_t s_start[kFB], s_end[kFB], lcur[kFB];
    __shared__ double tmp_d[16];
    __shared__ uint32_t tmp_u[16];
    __shared__ uint32_t s_key;
    __shared__ int s_top, s_first;
    __shared__ double s_tot;
    const int w = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, S = rs.S;
    const float *row = rs.row(r);
    const int c0 = w * rs.C, c1 = min(rs.V, c0 + rs.C);
    float v[kLoads];
    preload(row, c0, c1, v);
    const FStat *st = ws.fs + r * kMaxChunks;
    if (tid < 64) {   // the row's largest key, its top bin and e-mass (a lane a chunk)
        const uint32_t k = lane < S ? st[lane].key : 0u;
        const int tp = lane < S ? st[lane].top : INT_MIN;
        const float m = lane < S ? st[lane].mass : 0.0f;
        uint32_t mk = k;
        int mt = tp;
        for (int o = 32; o > 0; o >>= 1) {
            mk = max(mk, static_cast<uint32_t>(__shfl_xor(mk, o, 64)));
            mt = max(mt, __shfl_xor(mt, o, 64));
        }
        const float M = key_val(mk);
        const float sc = lane < S ? expf(__fdiv_rn(__fsub_rn(key_val(k), M), T)) : 0.0f;
        double tot = static_cast<double>(m) * static_cast<double>(sc);
        for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
        if (lane < S) {
            sscale[lane] = sc;
            soff[lane] = mt - tp;
        }
        if (lane == 0) {
            s_key = mk;
            s_top = mt;
            s_tot = tot;
            s_first = INT_MAX;
        }
    }
    __syncthreads();
    const float M = key_val(s_key);
    // the row's bin j (from its top): every chunk's bin j - (its offset), thread j + 64 h taking chunks h, h + 4, ..
    // (their loads all issued at once), the four quarters added in LDS; also the counts of the chunks before this one
    // (this chunk's first slot in each bin after the bin's start)
    double bw = 0.0;
    uint32_t bc = 0, bb = 0;
    {
        const int j = tid & 63, h = tid >> 6;
        uint32_t cc[kMaxChunks / 4];
        float ww[kMaxChunks / 4];
#pragma unroll
        for (int q = 0; q < kMaxChunks / 4; ++q) {
            const int c = min(4 * q + h, S - 1), jj = min(max(j - soff[c], 0), kFB - 1);
            cc[q] = st[c].cnt[jj];
            ww[q] = MASS ? st[c].w[jj] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < kMaxChunks / 4; ++q) {
            const int c = 4 * q + h, jl = j - soff[min(c, S - 1)];
            const bool in = c < S && j < kFB && jl >= 0 && jl < kFB;
            bc += in ? cc[q] : 0u;
            bb += in && c < w ? cc[q] : 0u;
            if (MASS) bw += in ? static_cast<double>(ww[q]) * static_cast<double>(sscale[c]) : 0.0;
        }
        sq_c[h][j] = bc;
        sq_b[h][j] = bb;
        sq_w[h][j] = bw;
        __syncthreads();
        bc = tid < kFB ? (sq_c[0][tid] + sq_c[1][tid]) + (sq_c[2][tid] + sq_c[3][tid]) : 0u;
        bb = tid < kFB ? (sq_b[0][tid] + sq_b[1][tid]) + (sq_b[2][tid] + sq_b[3][tid]) : 0u;
        bw = tid < kFB ? (sq_w[0][tid] + sq_w[1][tid]) + (sq_w[2][tid] + sq_w[3][tid]) : 0.0;
    }
    bool hit;
    uint32_t ctot;
    const uint32_t cex = block_excl_scan(bc, tmp_u, ctot);
    if (MASS) {
        double wtot;
        const double wex = block_excl_scan(bw, tmp_d, wtot);
        hit = tid < kFB && wex + bw >= static_cast<double>(top_p) * s_tot * (1.0 + 1e-3);
    } else {
        hit = tid < kFB && cex + bc >= static_cast<uint32_t>(K);
    }
    wave_min_hit(hit, tid, &s_first);
    if (tid < kFB) {   // bin j's elements go to [cex, cex + bc) of the row's list (the counts are whole for j <= jc),
        s_start[tid] = cex + bb;   // this chunk's from cex + bb
        s_end[tid] = cex + bc;
        lcur[tid] = 0u;
    }
    __syncthreads();
    const bool ok = isfinite(M) && s_first != INT_MAX;
    const int jc = MASS ? min(s_first + 1, kFB - 1) : s_first;
    const int thr = ok ? s_top - jc : INT_MAX;   // collected: row bin s_top - fbin(l) <= jc
    const float s4 = 4.0f / T;
    double part = 0.0;
    uint64_t *cand = ws.cand + static_cast<int64_t>(r) * kMaxCand;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        const int i = c0 + u * kPass + tid;
        if (i >= c1) continue;
        if (MASS) part += static_cast<double>(e_of(v[u], M, T));
        const int b = fbin(v[u], s4);
        if (b < thr) continue;
        const int j = s_top - b;
        const uint32_t at = s_start[j] + atomicAdd(&lcur[j], 1u);
        if (at < static_cast<uint32_t>(kFCap)) cand[at] = comp_of(v[u], static_cast<uint32_t>(i));
    }
    if (MASS) {
        const double cs = block_sum(part, tmp_d);
        if (tid == 0) ws.psum[r * kMaxChunks + w] = cs;
    }
    if (w == 0) {   // the row's bins' counts, for the nucleus
        if (tid < kFB) ws.fbc[r * kFB + tid] = ok && tid <= jc ? s_end[tid] - (s_start[tid] - bb) : 0u;
        if (tid == 0) {
            ws.fr[r].ok = ok;
            ws.fr[r].n = ok ? s_end[jc] : 0u;
            ws.fr[r].top_key = s_key;
            ws.fr[r].jc = jc;
        }
    }
}

// Elements sorted by rank within their groups: in[g0, g1) is group g's, every key distinct; the element at i goes to
// out[g0 + (how many of its group order before it)] (before: a greater key when DESC, a smaller one otherwise).
// find(i) gives i's group bounds. Every thread of the workgroup; the caller synchronises after.
template <bool DESC, typename Find>
__device__ inline void rank_place(const uint64_t *in, uint64_t *out, int n, Find find) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t c = in[i];
        uint32_t g0, g1;
        find(i, c, g0, g1);
        uint32_t rk[8] = {};   // (eight loads in flight)
        uint32_t j = g0;
        for (; j + 8 <= g1; j += 8)
#pragma unroll
            for (int q = 0; q < 8; ++q) rk[q] += DESC ? in[j + q] > c : in[j + q] < c;
        for (; j < g1; ++j) rk[0] += DESC ? in[j] > c : in[j] < c;
        out[g0 + ((rk[0] + rk[1]) + (rk[2] + rk[3])) + ((rk[4] + rk[5]) + (rk[6] + rk[7]))] = c;
    }
}

// A workgroup a row: the reference's nucleus (sampler.cpp:31-49) on the collected elements, which arrive grouped by
// bin, the bins in the sorted order: e_i = exp((l_i - max) / T); sum = every element's e (the chunks' sums in order);
// keep = the first i (in the sorted order) where the running sum over sum reaches top_p; kept = e_0 + .. +
// e_{keep-1}; the draw of u[row]: the first i < keep where kept u - (e_0 + .. + e_i) <= 0. One scan over the grouped
// elements gives the running sum at every bin's end, which does not depend on the order inside the bins; only the bin
// where top_p is reached and the bin where the draw lands are put in order (by rank) and scanned again. A row whose
// prefix does not end inside the collected elements is marked undecided.
constexpr int kSeg = kFCap / kSortThreads;   // consecutive elements a thread scans

// inclusive running sums of v over positions [0, m) (m <= kFCap, thread t taking t kSeg ..); cl[j]: through position
// t kSeg + j (tmp: LDS of 16 doubles); the total
__device__ inline double seg_scan(const double (&v)[kSeg], double (&cl)[kSeg], double *tmp) {
    double loc = 0.0;
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
        loc += v[j];
        cl[j] = loc;
    }
    double tot;
    const double ex = block_excl_scan(loc, tmp, tot);
#pragma unroll
    for (int j = 0; j < kSeg; ++j) cl[j] += ex;
    return tot;
}

// how many of in[j0 + G i] < in[j1] exceed c (eight loads in flight)
__device__ inline uint32_t count_above(const uint64_t *in, int j0, int j1, int G, uint64_t c) {
    uint32_t rk[8] = {};
    int j = j0;
    for (; j + 7 * G < j1; j += 8 * G)
#pragma unroll
        for (int q = 0; q < 8; ++q) rk[q] += in[j + q * G] > c;
    for (; j < j1; j += G) rk[0] += in[j] > c;
    return ((rk[0] + rk[1]) + (rk[2] + rk[3])) + ((rk[4] + rk[5]) + (rk[6] + rk[7]));
}


// in[g, g + m) put in descending order into out[0, m) by rank (keys distinct); every thread of the workgroup; the
// caller synchronises. Up to half the threads' count of elements: G adjacent lanes an element, lane q counting the
// others at q, q + G, .. (adjacent words for adjacent lanes: no LDS bank conflicts), their counts added across them.
__device__ inline void rank_sort_desc(const uint64_t *in, int g, int m, uint64_t *out) {
    const int tid = threadIdx.x, nthr = blockDim.x;
    if (2 * m <= nthr) {
        int lg = 1;   // G = 2^lg lanes an element
        while ((2 << lg) * m <= nthr && lg < 6) ++lg;
        const int G = 1 << lg, i = tid >> lg, q = tid & (G - 1);
        const uint64_t c = i < m ? in[g + i] : 0ull;
        uint32_t rk = i < m ? count_above(in, g + q, g + m, G, c) : 0u;
        for (int o = 1; o < G; o <<= 1) rk += __shfl_xor(rk, o, 64);
        if (i < m && q == 0) out[rk] = c;
        return;
    }
    for (int i = tid; i < m; i += nthr) {
        const uint64_t c = in[g + i];
        out[count_above(in, g, g + m, 1, c)] = c;
    }
}

// The first position p < m where pred(base + v(0) + .. + v(p)) holds, into s_pos (INT_MAX: none), the running sum
// there into s_cum; every thread of the workgroup, synchronised on return. Up to 512 positions one wave scans them
// (eight a lane); more (up to kFCap) the workgroup.
template <typename Val, typename Pred>
__device__ void first_reach(int m, double base, Val val, Pred pred, double *tmp, int &s_pos, double &s_cum) {
    const int tid = threadIdx.x;
    if (tid == 0) s_pos = INT_MAX;
    if (m <= 512) {
        if (tid < 64) {
            double cl[8], loc = 0.0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                loc += 8 * tid + j < m ? val(8 * tid + j) : 0.0;
                cl[j] = loc;
            }
            const double ex = base + wave_incl_scan(loc) - loc;
            int hit = -1;
            double at = 0.0;
#pragma unroll
            for (int j = 7; j >= 0; --j)
                if (8 * tid + j < m && pred(ex + cl[j])) {
                    hit = j;
                    at = ex + cl[j];
                }
            const uint64_t bal = __ballot(hit >= 0);
            if (bal && tid == __builtin_ctzll(bal)) {
                s_pos = 8 * tid + hit;
                s_cum = at;
            }
        }
        __syncthreads();
        return;
    }
    const int i0 = tid * kSeg;
    double v[kSeg], cl[kSeg];
#pragma unroll
    for (int j = 0; j < kSeg; ++j) v[j] = i0 + j < m ? val(i0 + j) : 0.0;
    (void)seg_scan(v, cl, tmp);
    int hit = INT_MAX;
#pragma unroll
    for (int j = kSeg - 1; j >= 0; --j)
        if (i0 + j < m && pred(base + cl[j])) hit = i0 + j;
    wave_min_hit(hit != INT_MAX, hit, &s_pos);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSeg; ++j)
        if (i0 + j == s_pos) s_cum = base + cl[j];
    __syncthreads();
}

template <bool MASS>
__global__ __launch_bounds__(kSortThreads) void fast_nucleus(Rows rs, Ws ws, float T, float top_p, int K, FastU fu) {
    extern __shared__ uint64_t lds[];   // [kFCap] the collected elements (by bin), [kFCap] doubles: the running e
                                        // sums, [kFCap] the bins put in order, each at its own place
    uint64_t *in = lds, *srt = lds + 2 * kFCap;
    double *cum = reinterpret_cast<double *>(lds + kFCap);
    __shared__ uint32_t s_start[kFB + 1];
    __shared__ double tmp_d[16];
    __shared__ double e_part[kMaxChunks];
    __shared__ int s_bk, s_bd, s_t, s_td;
    __shared__ double s_sum, s_kept, s_dcum;
    __shared__ unsigned long long s_max;
    const int r = blockIdx.x, tid = threadIdx.x;
    FRow &fr = ws.fr[r];
    const int n = static_cast<int>(fr.n), jc = fr.jc;
    if (!fr.ok || n <= 0 || n > kFCap || (MASS ? !(top_p < 1.0f) : n < K)) {
        if (tid == 0) fr.ok = 0;
        return;
    }
    uint64_t *cand = ws.cand + static_cast<int64_t>(r) * kMaxCand;
    const float mx = key_val(fr.top_key);
    if (tid < 64) {   // the bins' starts (wave 0)
        const uint32_t c = tid < kFB ? ws.fbc[r * kFB + tid] : 0u;
        const uint32_t incl = wave_incl_scan(c);
        if (tid < kFB) s_start[tid] = incl - c;
        if (tid == kFB - 1) s_start[kFB] = incl;
    }
    if (MASS && tid < rs.S) e_part[tid] = ws.psum[r * kMaxChunks + tid];
    for (int i = tid; i < n; i += blockDim.x) in[i] = cand[i];
    __syncthreads();
    // the top K (count mode): the bins before the last one, then the last one's first K - (its start) in order
    const int Kc = MASS ? n : K, gj = static_cast<int>(s_start[jc]);
    if (!MASS) {
        rank_sort_desc(in, gj, static_cast<int>(s_start[jc + 1]) - gj, srt + gj);
        __syncthreads();
    }
    auto e_at = [=](uint64_t c) { return static_cast<double>(e_of(key_val(static_cast<uint32_t>(c >> 32)), mx, T)); };
    const int i0 = tid * kSeg;
    double v[kSeg], cl[kSeg];
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
        const int p = i0 + j;
        v[j] = p < Kc ? e_at(!MASS && p >= gj ? srt[p] : in[p]) : 0.0;
    }
    const double tot = seg_scan(v, cl, tmp_d);
#pragma unroll
    for (int j = 0; j < kSeg; ++j)
        if (i0 + j < Kc) cum[i0 + j] = cl[j];
    if (MASS && tid == 0) {
        double t = 0.0;   // the row's e sum, chunks in order
        for (int c = 0; c < rs.S; ++c) t += e_part[c];
        s_sum = t;
    }
    __syncthreads();
    const double sum = MASS ? s_sum : tot, target = static_cast<double>(top_p);
    auto live = [&](int b) { return s_start[b + 1] > s_start[b] && static_cast<int>(s_start[b]) < Kc; };
    auto end_of = [&](int b) { return cum[min(static_cast<int>(s_start[b + 1]), Kc) - 1]; };   // (a live bin)
    auto before = [&](int b) { return s_start[b] ? cum[s_start[b] - 1] : 0.0; };
    auto sorted_e = [=](int g) { return [=](int p) { return e_at(srt[g + p]); }; };
    if (tid < 64) {   // the bin where the running sum reaches top_p
        const bool hit = top_p < 1.0f && tid < kFB && live(tid) && end_of(tid) / sum >= target;
        const uint64_t m = __ballot(hit);
        if (tid == 0) s_bk = m ? __builtin_ctzll(m) : -1;
    }
    __syncthreads();
    int bk = s_bk, t;
    double kept;
    if (bk < 0) {
        if (MASS) {   // the prefix goes on past the collected elements
            if (tid == 0) fr.ok = 0;
            return;
        }
        bk = jc;   // (count mode: top_p 1, or never reached: the whole top K kept)
        t = Kc - 1 - gj;
        kept = cum[Kc - 1];
    } else {
        const int gk = static_cast<int>(s_start[bk]), mk = min(static_cast<int>(s_start[bk + 1]), Kc) - gk;
        if (MASS || bk != jc) {
            rank_sort_desc(in, gk, static_cast<int>(s_start[bk + 1]) - gk, srt + gk);
            __syncthreads();
        }
        first_reach(mk, before(bk), sorted_e(gk), [=](double c) { return c / sum >= target; }, tmp_d, s_t, s_kept);
        if (s_t == INT_MAX) {   // (rounding: the bin's end in its sorted order fell short)
            if (tid == 0) fr.ok = 0;
            return;
        }
        t = s_t;
        kept = s_kept;
    }
    const int gk = static_cast<int>(s_start[bk]), keep = gk + t + 1;
    const double rr = kept * fu.u[r];
    if (tid < 64) {   // the draw's bin: the first before bk whose end reaches rr, else bk
        const bool hit = tid < bk && live(tid) && rr - end_of(tid) <= 0.0;
        const uint64_t m = __ballot(hit);
        if (tid == 0) s_bd = m ? __builtin_ctzll(m) : bk;
    }
    __syncthreads();
    const int bd = s_bd;
    uint64_t pick_c;
    const auto drawn = [=](double c) { return rr - c <= 0.0; };
    if (bd == bk) {
        first_reach(t + 1, before(bk), sorted_e(gk), drawn, tmp_d, s_td, s_dcum);
        pick_c = srt[gk + (s_td != INT_MAX ? s_td : t)];   // rounding past the end: the last kept
    } else {   // (bd < bk <= jc: a whole bin)
        const int gd = static_cast<int>(s_start[bd]), md = static_cast<int>(s_start[bd + 1]) - gd;
        rank_sort_desc(in, gd, md, srt + gd);
        __syncthreads();
        first_reach(md, before(bd), sorted_e(gd), drawn, tmp_d, s_td, s_dcum);
        if (s_td != INT_MAX) {
            pick_c = srt[gd + s_td];
        } else {   // (rounding: the bin's end in its sorted order fell short) the next live bin's first element
            int b2 = bd + 1;
            while (!live(b2)) ++b2;   // (bk is live)
            if (b2 == bk) {
                pick_c = srt[gk];
            } else {
                if (tid == 0) s_max = 0ull;
                __syncthreads();
                for (int i = static_cast<int>(s_start[b2]) + tid; i < static_cast<int>(s_start[b2 + 1]); i += blockDim.x)
                    atomicMax(&s_max, static_cast<unsigned long long>(in[i]));
                __syncthreads();
                pick_c = s_max;
            }
        }
    }
    if (tid == 0) {
        const int32_t pick = static_cast<int32_t>(comp_index(pick_c));
        RowInfo &info = ws.info[r];
        info.mx = mx;
        info.sum = sum;
        info.keep = static_cast<uint32_t>(keep);
        info.kept = kept;
        info.pick = pick;
        ws.picks[r] = pick;
        fr.last = srt[gk + t];
    }
    if (MASS)   // the kept prefix for the residual: the bins before bk stay as collected, then bk's first t + 1
        for (int i = tid; i <= t; i += blockDim.x) cand[gk + i] = srt[gk + i];
}

// The textbook rule over the candidate path's nuclei (target rows 0..k, draft rows k+1..2k; one workgroup): as
// textbook_finish, with p(x) and q(x) read from the kept prefixes. At a rejection the target's kept prefix (p is 0
// elsewhere) is put in index order by 256 buckets of indices and ranks within them, its residuals summed by one scan.
// st[0] = emitted, or 0 when a row was not decided here (out untouched).
constexpr int kBuckets = 256;
constexpr int kRankMax = 512;   // a bucket of more elements is sorted by the bitonic network instead

__global__ __launch_bounds__(kSortThreads) void fast_textbook(Rows rs, Ws ws, int k, float T, FastU fu,
                                                              int32_t *__restrict__ out, int *__restrict__ st,
                                                              uint32_t *done, uint32_t seq) {
    extern __shared__ uint64_t lds[];   // [kFCap] (index << 32) | position by bucket, [kFCap] in index order,
                                        // [kFCap] doubles: the residuals by position
    uint64_t *grp = lds, *ord = lds + kFCap;
    double *res = reinterpret_cast<double *>(lds + 2 * kFCap);
    __shared__ uint32_t bcnt[kBuckets], bstart[kBuckets + 1], bcur[kBuckets];
    __shared__ uint32_t tmp_u[16];
    __shared__ double tmp_d[16];
    __shared__ int s_rej, s_first, s_last, s_big;
    const int tid = threadIdx.x, nthr = blockDim.x, R = 2 * k + 1;
    if (tid < 64) {
        const uint64_t bad = __ballot(tid < R && ws.fr[min(tid, R - 1)].ok == 0);
        if (tid == 0) s_rej = bad ? -1 : INT_MAX;
    }
    if (tid < kBuckets) {
        bcnt[tid] = 0u;
        bcur[tid] = 0u;
    }
    // the results: out[0, n - 1) the stood drafts, out[n - 1] = last, st[0] = n, then the posting (post_seq)
    auto emit = [&](int n, int32_t last) {
        for (int i = tid; i < n - 1; i += nthr) out[i] = ws.picks[k + 1 + i];
        __threadfence_system();
        __syncthreads();
        if (tid == 0) {
            out[n - 1] = last;
            st[0] = n;
            post_seq(done, seq);
        }
    };
    __syncthreads();
    if (s_rej < 0) {
        if (tid == 0) {
            st[0] = 0;
            post_seq(done, seq);
        }
        return;
    }
    if (tid < k) {   // draft i stands with probability min(1, p_i(d) / q_i(d))
        const int i = tid, d = ws.picks[k + 1 + i];
        const RowInfo &P = ws.info[i], &Q = ws.info[k + 1 + i];
        const float lq = rs.row(k + 1 + i)[d], lp = rs.row(i)[d];
        const double qd = static_cast<double>(e_of(lq, Q.mx, T)) / Q.kept;
        const bool in_p = comp_of(lp, static_cast<uint32_t>(d)) >= ws.fr[i].last;
        const double pd = in_p ? static_cast<double>(e_of(lp, P.mx, T)) / P.kept : 0.0;
        if (!(static_cast<double>(fu.acc[i]) * qd < pd)) atomicMin(&s_rej, i);
    }
    __syncthreads();
    const int rej = s_rej;
    if (rej == INT_MAX) {   // every draft stood: the bonus, target row k's draw
        emit(k + 1, ws.picks[k]);
        return;
    }
    const RowInfo &P = ws.info[rej], &Q = ws.info[k + 1 + rej];
    const int keep = static_cast<int>(P.keep);
    const uint64_t *pc = ws.cand + static_cast<int64_t>(rej) * kMaxCand;
    const float *tq = rs.row(k + 1 + rej);
    const uint64_t lastq = ws.fr[k + 1 + rej].last;
    const float bscale = static_cast<float>(kBuckets) / static_cast<float>(rs.V);
    auto bucket = [&](uint32_t x) { return min(static_cast<int>(static_cast<float>(x) * bscale), kBuckets - 1); };
    for (int j = tid; j < keep; j += nthr) {   // max(0, p - q) of the kept prefix's element j; its bucket counted
        const uint64_t c = pc[j];
        const uint32_t x = comp_index(c);
        const float lq = tq[x];
        const double p = static_cast<double>(e_of(key_val(static_cast<uint32_t>(c >> 32)), P.mx, T)) / P.kept;
        const double q = comp_of(lq, x) >= lastq ? static_cast<double>(e_of(lq, Q.mx, T)) / Q.kept : 0.0;
        res[j] = fmax(0.0, p - q);
        ord[j] = (static_cast<uint64_t>(x) << 32) | static_cast<uint32_t>(j);
        atomicAdd(&bcnt[bucket(x)], 1u);
    }
    __syncthreads();
    {
        const uint32_t c = tid < kBuckets ? bcnt[tid] : 0u;
        uint32_t tot;
        const uint32_t ex = block_excl_scan(c, tmp_u, tot);
        if (tid < kBuckets) bstart[tid] = ex;
        if (tid == 0) {
            bstart[kBuckets] = tot;
            s_big = 0;
        }
        __syncthreads();
        if (c > static_cast<uint32_t>(kRankMax)) s_big = 1;
    }
    for (int j = tid; j < keep; j += nthr) {   // grouped by bucket
        const uint64_t o = ord[j];
        const int b = bucket(static_cast<uint32_t>(o >> 32));
        grp[bstart[b] + atomicAdd(&bcur[b], 1u)] = o;
    }
    __syncthreads();
    if (!s_big) {
        rank_place<false>(grp, ord, keep, [&](int, uint64_t c, uint32_t &g0, uint32_t &g1) {
            const int b = bucket(static_cast<uint32_t>(c >> 32));
            g0 = bstart[b];
            g1 = bstart[b + 1];
        });
        __syncthreads();
    } else {   // (index ascending: ~index descending)
        int Pn = 1;
        while (Pn < keep) Pn <<= 1;
        for (int j = tid; j < Pn; j += nthr)
            ord[j] = j < keep ? (grp[j] ^ 0xFFFFFFFF00000000ull) : 0ull;
        __syncthreads();
        bitonic_desc(ord, Pn);
        for (int j = tid; j < keep; j += nthr) ord[j] ^= 0xFFFFFFFF00000000ull;
        __syncthreads();
    }
    const int i0 = tid * kSeg;
    double rv[kSeg], cl[kSeg];
    double loc = 0.0;
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
        rv[j] = i0 + j < keep ? res[static_cast<uint32_t>(ord[i0 + j])] : 0.0;
        loc += rv[j];
        cl[j] = loc;
    }
    double total;
    const double ex = block_excl_scan(loc, tmp_d, total);
    int pick;
    if (!(total > 0.0)) {
        pick = ws.picks[rej];   // no residual mass: the target row's own draw
    } else {
        const double goal = static_cast<double>(fu.res) * total;
        if (tid == 0) {
            s_first = INT_MAX;
            s_last = -1;
        }
        __syncthreads();
        int last = -1, first = INT_MAX;
#pragma unroll
        for (int j = 0; j < kSeg; ++j)
            if (rv[j] > 0.0) last = i0 + j;
#pragma unroll
        for (int j = kSeg - 1; j >= 0; --j)
            if (rv[j] > 0.0 && cl[j] + ex >= goal) first = i0 + j;
        wave_max_hit(last >= 0, last, &s_last);
        wave_min_hit(first != INT_MAX, first, &s_first);
        __syncthreads();
        const int at = s_first != INT_MAX ? s_first : s_last;   // rounding past the end: the last positive weight
        pick = static_cast<int>(ord[at] >> 32);
    }
    emit(rej + 1, pick);
}

// The textbook rule when greedy (target rows 0..k, draft rows k+1..2k; one workgroup, their chunks' maxima done):
// each row's first argmax from its chunks' (a wave a row), then target row i's argmax is emitted while draft row i's
// agrees, and target row k's when all do (the bonus). st[0] = emitted, then seq to *done (post_seq).
__global__ __launch_bounds__(kSortThreads) void greedy_finish(Ws ws, int S, int k, int32_t *__restrict__ out,
                                                              int *__restrict__ st, uint32_t *done, uint32_t seq) {
    __shared__ int32_t pick[64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, R = 2 * k + 1;
    for (int r = wave; r < R; r += blockDim.x >> 6) {
        uint64_t best = 0;
        if (lane < S)
            best = (static_cast<uint64_t>(ws.pmax[r * kMaxChunks + lane]) << 32) |
                   (0xFFFFFFFFu - static_cast<uint32_t>(ws.pidx[r * kMaxChunks + lane]));
        for (int o = 32; o > 0; o >>= 1) best = max(best, static_cast<uint64_t>(__shfl_xor(best, o, 64)));
        if (lane == 0) pick[r] = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(best));
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    int emitted = 0;
    for (int i = 0; i < k; ++i) {
        out[emitted++] = pick[i];
        if (pick[i] != pick[k + 1 + i]) {
            st[0] = emitted;
            post_seq(done, seq);
            return;
        }
    }
    out[emitted++] = pick[k];
    st[0] = emitted;
    post_seq(done, seq);
}

// ---------------------------------------------------------------- host side
struct Workspace {
    void *p = nullptr;
    size_t n = 0;
    void *get(size_t want) {
        if (want <= n) return p;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        if (hipMalloc(&p, want) != hipSuccess) return nullptr;
        n = want;
        return p;
    }
};

// pinned host memory for a call's inputs and results (one copy each way, or the results written by the kernels),
// coherent: the kernels' system-scope stores reach the host while the stream still runs
struct Pinned {
    void *p = nullptr;
    size_t n = 0;
    void *get(size_t want) {
        if (want <= n) return p;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
        if (hipHostMalloc(&p, want, hipHostMallocCoherent) != hipSuccess) return nullptr;
        n = want;
        return p;
    }
};

std::atomic<int64_t> g_path_candidate{0}, g_path_walks{0};   // the acceptance rules' sampling calls by path

// A call's sequence number (never 0), its word in pinned memory cleared for it before the launches
std::atomic<uint32_t> g_seq{0};
uint32_t next_seq(uint32_t *done) {
    uint32_t s = g_seq.fetch_add(1, std::memory_order_relaxed) + 1;
    if (s == 0) s = g_seq.fetch_add(1, std::memory_order_relaxed) + 1;
    __atomic_store_n(done, 0u, __ATOMIC_RELAXED);
    return s;
}

// Waits until the call's last kernel has posted seq at *done (post_seq: its results in the same pinned buffer are
// visible by then), polling the word: the stream wait returns several microseconds after the kernel is done. Once the
// wait has lasted kQueryAfterUs, the stream is queried every 1024 polls, so a failed launch or a fault ends the wait
// with its error, and a stream that finished without posting is an error too. (Queries from the start cost a short
// call ~10 us: measured 31-35 us a greedy textbook trial against 17 us.)
constexpr int64_t kQueryAfterUs = 10000;
int wait_posted(const uint32_t *done, uint32_t seq, hipStream_t st) {
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t n = 1;; ++n) {
        if (__atomic_load_n(done, __ATOMIC_ACQUIRE) == seq) return 0;
        if ((n & 1023u) != 0) continue;
        if (std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() <
            kQueryAfterUs)
            continue;
        const hipError_t e = hipStreamQuery(st);
        if (e == hipErrorNotReady) continue;
        GV_CHECK_HIP(e);
        if (__atomic_load_n(done, __ATOMIC_ACQUIRE) == seq) return 0;
        GV_REQUIRE(false, "sampler: the stream finished without the call's posted results");
    }
}

Workspace &ws_mem() {
    static Workspace w;
    return w;
}
Pinned &pinned() {
    static Pinned p;
    return p;
}

constexpr size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// The arrays of R rows, carved from one allocation, then `io` bytes for the call's inputs and results: the inputs
// (the uniforms first, then the caller's) are copied in one piece from pinned memory, the results back likewise.
struct Carved {
    Ws ws;
    char *io;   // device: [R] doubles of uniforms, then the caller's arrays
};

size_t ws_bytes(int R, size_t io) {
    size_t b = 0;
    b += align256(sizeof(RowInfo) * R);
    b += align256(static_cast<size_t>(R) * kMaxChunks * 16);
    b += align256(sizeof(LevelHist) * kHists * R);
    b += align256(16 * static_cast<size_t>(R) + 4 * static_cast<size_t>(R));
    b += align256(static_cast<size_t>(R) * kMaxCand * 8);
    b += align256(static_cast<size_t>(R) * 2 * kList * 8);
    b += align256(sizeof(FStat) * kMaxChunks * R);
    b += align256(sizeof(FRow) * R);
    b += align256(4 * static_cast<size_t>(kFB) * R);
    b += align256(8 * static_cast<size_t>(R) + io);
    return b;
}

Carved carve(void *base, int R) {
    char *p = static_cast<char *>(base);
    Carved c{};
    Ws &w = c.ws;
    w.info = reinterpret_cast<RowInfo *>(p);
    p += align256(sizeof(RowInfo) * R);
    const size_t ch = static_cast<size_t>(R) * kMaxChunks;
    w.psum = reinterpret_cast<double *>(p);
    w.pmax = reinterpret_cast<uint32_t *>(p + ch * 8);
    w.pidx = reinterpret_cast<int32_t *>(p + ch * 12);
    p += align256(ch * 16);
    w.h = reinterpret_cast<LevelHist *>(p);
    p += align256(sizeof(LevelHist) * kHists * R);
    w.cnt = reinterpret_cast<uint32_t *>(p);
    w.picks = reinterpret_cast<int32_t *>(p + 16 * static_cast<size_t>(R));
    p += align256(16 * static_cast<size_t>(R) + 4 * static_cast<size_t>(R));
    w.cand = reinterpret_cast<uint64_t *>(p);
    p += align256(static_cast<size_t>(R) * kMaxCand * 8);
    w.lst = reinterpret_cast<uint64_t *>(p);
    p += align256(static_cast<size_t>(R) * 2 * kList * 8);
    w.fs = reinterpret_cast<FStat *>(p);
    p += align256(sizeof(FStat) * kMaxChunks * R);
    w.fr = reinterpret_cast<FRow *>(p);
    p += align256(sizeof(FRow) * R);
    w.fbc = reinterpret_cast<uint32_t *>(p);
    p += align256(4 * static_cast<size_t>(kFB) * R);
    c.io = p;
    w.u = reinterpret_cast<double *>(p);
    return c;
}

Rows make_rows(const float *x1, int R1, const float *x2, int64_t ld, int V) {
    Rows rs{x1, x2, ld, R1, V, 1, V};
    rs.S = std::max(1, (V + kChunk - 1) / kChunk);
    rs.C = (V + rs.S - 1) / rs.S;
    rs.S = (V + rs.C - 1) / rs.C;   // (no empty chunk)
    return rs;
}

template <int KP>
int launch_cand_nucleus(const Rows &rs, const Ws &ws, int R, float T, float top_p, hipStream_t st) {
    static int granted = 0;
    const size_t lds = static_cast<size_t>(KP) * 8;
    if (lds_grant(reinterpret_cast<const void *>(&cand_nucleus<KP>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(cand_nucleus<KP>, dim3(R), dim3(kSortThreads), lds, st, rs, ws, T, top_p);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// The pick of each of R rows into ws.picks (and, sampling, its nucleus into ws.info), the uniforms already in ws.u:
// T <= 0 the first argmax; top_k or cap below V the top-K candidates' nucleus (K <= 16384); else the full
// vocabulary's.
int nuclei(const Rows &rs, int R, float T, float top_p, int top_k, int cap, const Ws &ws, hipStream_t st) {
    GV_REQUIRE(rs.S <= kMaxChunks, "sampler: a vocabulary of at most 262,144 tokens");
    const dim3 grid(rs.S, R), block(kPass);
    if (T <= 0.0f) {
        hipLaunchKernelGGL(max_pass<false>, grid, block, 0, st, rs, ws);
        hipLaunchKernelGGL(argmax_reduce, dim3(R), dim3(64), 0, st, ws, rs.S);
        GV_CHECK_HIP(hipGetLastError());
        return 0;
    }
    hipLaunchKernelGGL(max_pass<true>, grid, block, 0, st, rs, ws);
    const int K = top_k > 0 ? std::min(top_k, rs.V) : (cap > 0 ? std::min(cap, rs.V) : rs.V);
    if (K < rs.V) {   // the top-K candidates: a count walk to the K-th, collected, sorted, the nucleus as written
        GV_REQUIRE(K <= kMaxCand, "sampler: at most 16384 top-k candidates (top_k or cap); 0 takes the whole vocabulary");
        hipLaunchKernelGGL(level1_pass<false>, grid, block, 0, st, rs, ws, T);
        hipLaunchKernelGGL((walk_pass<false, ST_P1>), grid, block, 0, st, rs, ws, T, top_p, K);
        hipLaunchKernelGGL((walk_pass<false, ST_P2>), grid, block, 0, st, rs, ws, T, top_p, K);
        GV_CHECK_HIP(hipGetLastError());
        return K <= 1024 ? launch_cand_nucleus<1024>(rs, ws, R, T, top_p, st)
             : K <= 4096 ? launch_cand_nucleus<4096>(rs, ws, R, T, top_p, st)
                         : launch_cand_nucleus<kMaxCand>(rs, ws, R, T, top_p, st);
    }
    // every token a candidate: the mass walks over the whole row, no sort
    hipLaunchKernelGGL(level1_pass<true>, grid, block, 0, st, rs, ws, T);
    hipLaunchKernelGGL((walk_pass<true, ST_P1>), grid, block, 0, st, rs, ws, T, top_p, K);
    hipLaunchKernelGGL((walk_pass<true, ST_P2>), grid, block, 0, st, rs, ws, T, top_p, K);
    hipLaunchKernelGGL((walk_pass<true, ST_D1>), grid, block, 0, st, rs, ws, T, top_p, K);
    hipLaunchKernelGGL((walk_pass<true, ST_D2>), grid, block, 0, st, rs, ws, T, top_p, K);
    hipLaunchKernelGGL(draw_pick, dim3(R), block, 0, st, rs, ws, T);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace
}  // namespace gv

using namespace gv;

extern "C" {

int gv_sampler_paths(int64_t *candidate, int64_t *walks) {
    GV_REQUIRE(candidate && walks, "gv_sampler_paths: null argument");
    *candidate = g_path_candidate.load(std::memory_order_relaxed);
    *walks = g_path_walks.load(std::memory_order_relaxed);
    return 0;
}

int gv_sample_rows(const float *logits, int64_t ld, int rows, int V, float temperature, float top_p, int top_k,
                   int cap, const double *u, int32_t *out) {
    GV_REQUIRE(V <= kMaxVocab, "gv_sample_rows: a vocabulary of at most 262,144 tokens");
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(logits && out && rows >= 1 && rows <= kSampleRows && V >= 1 && ld >= V, "gv_sample_rows: bad arguments");
    GV_REQUIRE(temperature <= 0.0f || u, "gv_sample_rows: uniforms needed when temperature > 0");
    void *base = ws_mem().get(ws_bytes(rows, 0));
    auto *pin = static_cast<char *>(pinned().get(8 * static_cast<size_t>(rows)));
    GV_REQUIRE(base && pin, "gv_sample_rows: out of memory");
    const Carved c = carve(base, rows);
    const hipStream_t st = stream();
    if (temperature > 0.0f) {
        std::copy(u, u + rows, reinterpret_cast<double *>(pin));
        GV_CHECK_HIP(hipMemcpyAsync(c.ws.u, pin, 8 * static_cast<size_t>(rows), hipMemcpyHostToDevice, st));
    }
    const Rows rs = make_rows(logits, rows, nullptr, ld, V);
    if (nuclei(rs, rows, temperature, top_p, top_k, cap, c.ws, st) != 0) return -1;
    GV_CHECK_HIP(hipMemcpyAsync(pin, c.ws.picks, 4 * static_cast<size_t>(rows), hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    std::copy(reinterpret_cast<int32_t *>(pin), reinterpret_cast<int32_t *>(pin) + rows, out);
    return 0;
}

int gv_accept_match(const float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature,
                    float top_p, int top_k, int cap, const double *u, int32_t *out, int *kept) {
    // (no penalty: the rows are only read)
    return gv_accept_match_ex(const_cast<float *>(logits), ld, V, batch, n, temperature, top_p, top_k, cap, u, nullptr,
                              0, 0.0f, nullptr, 0, out, kept);
}

int gv_accept_match_ex(float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature, float top_p,
                       int top_k, int cap, const double *u, const int32_t *seen, int n_seen, float presence_penalty,
                       const int32_t *stop, int n_stop, int32_t *out, int *kept) {
    GV_REQUIRE(V <= kMaxVocab, "gv_accept_match: a vocabulary of at most 262,144 tokens");
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(logits && batch && out && n >= 1 && n <= 32 && V >= 1 && ld >= V, "gv_accept_match: bad arguments");
    GV_REQUIRE(temperature <= 0.0f || u, "gv_accept_match: uniforms needed when temperature > 0");
    GV_REQUIRE(n_seen >= 0 && (n_seen == 0 || seen) && n_seen <= V, "gv_accept_match: seen tokens");
    GV_REQUIRE(n_stop >= 0 && n_stop <= 1024 && (n_stop == 0 || stop), "gv_accept_match: at most 1024 stop tokens");
    const bool penalize = presence_penalty != 0.0f;
    // which drafts are new to the answer (one subtraction a token); seen must hold distinct tokens of the vocabulary
    int32_t fresh[33] = {};
    if (penalize) {
        std::vector<uint8_t> in(static_cast<size_t>(V), 0);
        for (int j = 0; j < n_seen; ++j) {
            GV_REQUIRE(seen[j] >= 0 && seen[j] < V && !in[static_cast<size_t>(seen[j])],
                       "gv_accept_match: seen tokens must be distinct tokens of the vocabulary");
            in[static_cast<size_t>(seen[j])] = 1;
        }
        for (int j = 1; j < n; ++j) {
            GV_REQUIRE(batch[j] >= 0 && batch[j] < V, "gv_accept_match: draft out of range");
            if (!in[static_cast<size_t>(batch[j])]) fresh[j] = 1, in[static_cast<size_t>(batch[j])] = 1;
        }
    }
    // io: [n] uniforms (doubles), then out[32], res[4], batch[32], fresh[33], stop[n_stop], seen[n_seen] (int32)
    const int n_seen_dev = penalize ? n_seen : 0;
    const size_t ints = 32 + 4 + 32 + 33 + static_cast<size_t>(n_stop) + static_cast<size_t>(n_seen_dev);
    const size_t io = 8 * static_cast<size_t>(n) + 4 * ints;
    void *base = ws_mem().get(ws_bytes(n, io));
    auto *pin = static_cast<char *>(pinned().get(io));
    GV_REQUIRE(base && pin, "gv_accept_match: out of memory");
    const Carved c = carve(base, n);
    int32_t *hint = reinterpret_cast<int32_t *>(pin + 8 * static_cast<size_t>(n));
    int32_t *dint = reinterpret_cast<int32_t *>(c.io + 8 * static_cast<size_t>(n));
    if (temperature > 0.0f) std::copy(u, u + n, reinterpret_cast<double *>(pin));
    std::copy(batch, batch + n, hint + 36);
    std::copy(fresh, fresh + 33, hint + 68);
    if (n_stop) std::copy(stop, stop + n_stop, hint + 101);
    if (n_seen_dev) std::copy(seen, seen + n_seen_dev, hint + 101 + n_stop);
    const hipStream_t st = stream();
    const Rows rs = make_rows(logits, n, nullptr, ld, V);
    const int K = top_k > 0 ? std::min(top_k, V) : (cap > 0 ? std::min(cap, V) : V);
    const bool candidate = temperature > 0.0f && K < V && K <= kFCap && rs.S <= kMaxChunks;
    static int granted_n = 0;
    const size_t lds_n = static_cast<size_t>(kFCap) * 24;
    if (candidate && lds_grant(reinterpret_cast<const void *>(&fast_nucleus<false>), lds_n, granted_n) != 0) return -1;
    auto launch_candidate = [&](const FastU &fu) {
        const dim3 grid(rs.S, n), block(kPass);
        hipLaunchKernelGGL(fast_stats, grid, block, 0, st, rs, c.ws, temperature);
        hipLaunchKernelGGL(fast_collect<false>, grid, block, 0, st, rs, c.ws, temperature, top_p, K);
        hipLaunchKernelGGL(fast_nucleus<false>, dim3(n), dim3(kSortThreads), lds_n, st, rs, c.ws, temperature, top_p, K,
                           fu);
    };
    FastU fu{};
    if (temperature > 0.0f)
        for (int i = 0; i < n; ++i) fu.u[i] = u[i];
    if ((candidate || temperature <= 0.0f) && !penalize && n_stop <= 32) {
        // no penalty and few stop tokens: every input as kernel arguments and the results straight into the pinned
        // buffer, no copy either way (greedy: the chunks' maxima and the first argmaxes)
        MatchIn in{};
        std::copy(batch, batch + n, in.batch);
        if (n_stop) std::copy(stop, stop + n_stop, in.stop);
        uint32_t *done = reinterpret_cast<uint32_t *>(hint + 34);
        const uint32_t seq = next_seq(done);
        if (candidate) {
            launch_candidate(fu);
            hipLaunchKernelGGL(match_args_kernel, dim3(1), dim3(64), 0, st, c.ws.picks, in, n, n_stop, hint, hint + 32,
                               static_cast<const FRow *>(c.ws.fr), done, seq);
        } else {
            GV_REQUIRE(rs.S <= kMaxChunks, "sampler: a vocabulary of at most 262,144 tokens");
            hipLaunchKernelGGL(max_pass<false>, dim3(rs.S, n), dim3(kPass), 0, st, rs, c.ws);
            hipLaunchKernelGGL(greedy_match_kernel, dim3(1), dim3(64), 0, st, c.ws, rs.S, in, n, n_stop, hint, hint + 32,
                               done, seq);
        }
        GV_CHECK_HIP(hipGetLastError());
        if (wait_posted(done, seq, st) != 0) return -1;
        const int emitted = hint[32];
        if (emitted > 0) {
            for (int i = 0; i < emitted; ++i) out[i] = hint[i];
            if (kept) *kept = hint[33];
            if (candidate) g_path_candidate.fetch_add(1, std::memory_order_relaxed);
            return emitted;
        }
        // (a row the candidate path did not decide: the walks below, from the copied inputs)
        std::copy(batch, batch + n, hint + 36);
    }
    GV_CHECK_HIP(hipMemcpyAsync(c.io, pin, io, hipMemcpyHostToDevice, st));
    int32_t *dout = dint, *dres = dint + 32, *dbatch = dint + 36, *dfresh = dint + 68, *dstop = dint + 101;
    int32_t *dseen = dstop + n_stop;
    if (penalize) {
        hipLaunchKernelGGL(penalty_kernel, dim3(n), dim3(256), 0, st, logits, ld, dseen, n_seen_dev, dbatch, dfresh,
                           presence_penalty);
        GV_CHECK_HIP(hipGetLastError());
    }
    if (candidate && (penalize || n_stop > 32)) {
        // the candidate path over the top K; a row it does not decide sends the call to the walks (the penalty
        // already applied)
        launch_candidate(fu);
        hipLaunchKernelGGL(match_kernel, dim3(1), dim3(64), 0, st, c.ws.picks, dbatch, n, dstop, n_stop, dout, dres,
                           static_cast<const FRow *>(c.ws.fr));
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipMemcpyAsync(hint, dout, 36 * 4, hipMemcpyDeviceToHost, st));
        GV_CHECK_HIP(hipStreamSynchronize(st));
        const int emitted = hint[32];
        if (emitted > 0) {
            for (int i = 0; i < emitted; ++i) out[i] = hint[i];
            if (kept) *kept = hint[33];
            g_path_candidate.fetch_add(1, std::memory_order_relaxed);
            return emitted;
        }
    }
    if (temperature > 0.0f) g_path_walks.fetch_add(1, std::memory_order_relaxed);
    if (nuclei(rs, n, temperature, top_p, top_k, cap, c.ws, st) != 0) return -1;
    hipLaunchKernelGGL(match_kernel, dim3(1), dim3(64), 0, st, c.ws.picks, dbatch, n, dstop, n_stop, dout, dres,
                       static_cast<const FRow *>(nullptr));
    GV_CHECK_HIP(hipGetLastError());
    GV_CHECK_HIP(hipMemcpyAsync(hint, dout, 36 * 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    const int emitted = hint[32];
    for (int i = 0; i < emitted; ++i) out[i] = hint[i];
    if (kept) *kept = hint[33];
    return emitted;
}

int gv_accept_textbook(const float *target, const float *draft, int64_t ld, int V, int k, float temperature,
                       float top_p, int greedy, const float *u_draft, const float *u_acc, float u_res, int32_t *out) {
    GV_REQUIRE(V <= kMaxVocab, "gv_accept_textbook: a vocabulary of at most 262,144 tokens");
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(target && draft && out && k >= 1 && k <= 31 && V >= 1 && ld >= V, "gv_accept_textbook: bad arguments");
    GV_REQUIRE(greedy || (u_draft && u_acc && temperature > 0.0f), "gv_accept_textbook: uniforms and T > 0 needed");
    const int R = 2 * k + 1;
    // io: [R] uniforms, then rsum[kMaxChunks] (double), u_acc[32] (float), done, out[32], st (uint32 / int32), and
    // the posted sequence word (host side only)
    const size_t io = 8 * static_cast<size_t>(R) + 8 * kMaxChunks + 4 * 32 + 4 + 4 * 33 + 4;
    void *base = ws_mem().get(ws_bytes(R, io));
    auto *pin = static_cast<char *>(pinned().get(io));
    GV_REQUIRE(base && pin, "gv_accept_textbook: out of memory");
    const Carved c = carve(base, R);
    double *rsum = reinterpret_cast<double *>(c.io + 8 * static_cast<size_t>(R));
    float *dacc = reinterpret_cast<float *>(rsum + kMaxChunks);
    uint32_t *ddone = reinterpret_cast<uint32_t *>(dacc + 32);
    int32_t *dout = reinterpret_cast<int32_t *>(ddone + 1);
    int *dst = dout + 32;
    // target rows 0..k draw with u_res (row k's is the bonus; a rejected row with no residual mass falls back to its
    // own), draft rows with u_draft
    double *hu = reinterpret_cast<double *>(pin);
    for (int r = 0; r <= k; ++r) hu[r] = static_cast<double>(u_res);
    for (int i = 0; i < k; ++i) hu[k + 1 + i] = greedy ? 0.0 : static_cast<double>(u_draft[i]);
    float *hacc = reinterpret_cast<float *>(pin + 8 * static_cast<size_t>(R) + 8 * kMaxChunks);
    for (int i = 0; i < k; ++i) hacc[i] = greedy ? 0.0f : u_acc[i];
    *reinterpret_cast<uint32_t *>(hacc + 32) = 0u;   // the finishing count
    const hipStream_t st = stream();
    const Rows rs = make_rows(target, k + 1, draft, ld, V);
    int32_t *hout = reinterpret_cast<int32_t *>(hacc + 33);
    uint32_t *done = reinterpret_cast<uint32_t *>(hout + 33);
    if (greedy) {   // the chunks' maxima, then the first argmaxes and the decisions, straight into the pinned buffer
        GV_REQUIRE(rs.S <= kMaxChunks, "sampler: a vocabulary of at most 262,144 tokens");
        const uint32_t seq = next_seq(done);
        hipLaunchKernelGGL(max_pass<false>, dim3(rs.S, R), dim3(kPass), 0, st, rs, c.ws);
        hipLaunchKernelGGL(greedy_finish, dim3(1), dim3(kSortThreads), 0, st, c.ws, rs.S, k, hout, hout + 32, done,
                           seq);
        GV_CHECK_HIP(hipGetLastError());
        if (wait_posted(done, seq, st) != 0) return -1;
        const int emitted = hout[32];
        for (int i = 0; i < emitted; ++i) out[i] = hout[i];
        return emitted;
    }
    if (!greedy && top_p < 1.0f && rs.S <= kMaxChunks) {
        // the candidate path, its uniforms as kernel arguments; a row it does not decide sends the call to the walks
        FastU fu{};
        for (int r = 0; r < R; ++r) fu.u[r] = hu[r];
        for (int i = 0; i < k; ++i) fu.acc[i] = u_acc[i];
        fu.res = u_res;
        const dim3 grid(rs.S, R), block(kPass);
        hipLaunchKernelGGL(fast_stats, grid, block, 0, st, rs, c.ws, temperature);
        hipLaunchKernelGGL(fast_collect<true>, grid, block, 0, st, rs, c.ws, temperature, top_p, 0);
        static int granted_n = 0, granted_t = 0;
        const size_t lds_n = static_cast<size_t>(kFCap) * 24, lds_t = static_cast<size_t>(kFCap) * 24;
        if (lds_grant(reinterpret_cast<const void *>(&fast_nucleus<true>), lds_n, granted_n) != 0 ||
            lds_grant(reinterpret_cast<const void *>(&fast_textbook), lds_t, granted_t) != 0)
            return -1;
        const uint32_t seq = next_seq(done);
        hipLaunchKernelGGL(fast_nucleus<true>, dim3(R), dim3(kSortThreads), lds_n, st, rs, c.ws, temperature, top_p, 0,
                           fu);
        // (the results straight into the pinned buffer: no copy launch)
        hipLaunchKernelGGL(fast_textbook, dim3(1), dim3(kSortThreads), lds_t, st, rs, c.ws, k, temperature, fu, hout,
                           hout + 32, done, seq);
        GV_CHECK_HIP(hipGetLastError());
        if (wait_posted(done, seq, st) != 0) return -1;
        const int emitted = hout[32];
        if (emitted > 0) {
            for (int i = 0; i < emitted; ++i) out[i] = hout[i];
            g_path_candidate.fetch_add(1, std::memory_order_relaxed);
            return emitted;
        }
    }
    g_path_walks.fetch_add(1, std::memory_order_relaxed);
    GV_CHECK_HIP(hipMemcpyAsync(c.io, pin, io, hipMemcpyHostToDevice, st));
    const float Tn = greedy ? 0.0f : temperature;
    if (nuclei(rs, R, Tn, top_p, 0, 0, c.ws, st) != 0) return -1;
    hipLaunchKernelGGL(textbook_finish, dim3(greedy ? 1 : rs.S), dim3(kPass), 0, st, rs, c.ws, k, greedy, temperature,
                       dacc, u_res, rsum, ddone, dout, dst);
    GV_CHECK_HIP(hipGetLastError());
    GV_CHECK_HIP(hipMemcpyAsync(hout, dout, 33 * 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    const int emitted = hout[32];
    for (int i = 0; i < emitted; ++i) out[i] = hout[i];
    return emitted;
}

}  // extern "C"
