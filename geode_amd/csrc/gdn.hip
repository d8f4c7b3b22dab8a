// gdn.hip - the Gated DeltaNet layer of the verify step (engine/src/model.cpp:3497-3688) on gfx950: the causal
// depthwise conv with silu, the q / k L2 norms and gates, the delta rule on each value head's [dk][dv] state, the
// gated RMSNorm into the output projection's operands. The projections themselves are the step's q4 products
// (in_proj_qkv | in_proj_z as one matrix of two globals, out_proj) and the a / b rows the router kernel's bf16 dots.
//
// States live in slots: two sets of max_rows slots a layer, each slot one row's conv state and recurrent state. A
// verify reads the base slot (the state the last verify or keep left) and writes row t's states into slot t of the
// other set; a row starts from its parent's slot (the tree's), the first row from the base. The states as after any
// row stay until the next verify, so verify_keep (model.cpp:1617-1633: the states as after the last kept row) only
// names a new base slot. A recurrent-state slot is read back in the launch only by the thread that wrote it; a conv
// state slot not at all (a row's conv window comes from its ancestors' raw inputs and the base slot).
//
// One launch after the projections, three roles in workgroup order (producers first): the a / b dots of each row,
// the core workgroups (conv, norms, gates, delta rule) once their row's dots are in, and the gated norm of each row
// once every core workgroup is done; the data between them goes through sc1 loads and stores with per-workgroup
// flags (common.hpp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"

namespace gv {

namespace {

// fast_exp (engine/src/kernels.hpp:142-163): Cephes' expf - the reduction by ln 2 in two parts, a degree-6
// polynomial, 2^n by the exponent's bits; each operation rounded on its own, so the bits are the host's
__device__ inline float fast_exp(float x) {
    x = fminf(fmaxf(x, -87.0f), 88.0f);
    const float n = floorf(__fadd_rn(__fmul_rn(x, 1.44269504088896341f), 0.5f));
    float r = __fsub_rn(x, __fmul_rn(n, 0.693359375f));
    r = __fadd_rn(r, __fmul_rn(n, 2.12194440e-4f));
    float p = 1.9875691500e-4f;
    p = __fadd_rn(__fmul_rn(p, r), 1.3981999507e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 8.3334519073e-3f);
    p = __fadd_rn(__fmul_rn(p, r), 4.1665795894e-2f);
    p = __fadd_rn(__fmul_rn(p, r), 1.6666665459e-1f);
    p = __fadd_rn(__fmul_rn(p, r), 5.0000001201e-1f);
    p = __fadd_rn(__fadd_rn(__fmul_rn(__fmul_rn(p, r), r), r), 1.0f);
    const uint32_t bits = __float_as_uint(p) + (static_cast<uint32_t>(static_cast<int32_t>(n)) << 23);
    return __uint_as_float(bits);
}
__device__ inline float silu_fast(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, fast_exp(-x))); }   // kernels.hpp:165

constexpr int kMaxConvK = 8;
constexpr int kGdnThreads = 256;

// The recurrent state's device layout: value head vh's [dk][dv] in blocks of 16 columns; in a block, column
// j0 + 4 w + c is held by lanes c 16 .. c 16 + 15 of wave w of a core workgroup, lane part taking rows
// part rpt .. part rpt + rpt - 1 (rpt = dk / 16), those rows vec (= min(rpt, 4)) floats at a time, a wave's 64 lanes
// contiguous per load.
__host__ __device__ inline int64_t s_index(int vh, int i, int j, int dk, int dv) {
    const int rpt = dk / 16, vec = rpt < 4 ? rpt : 4;
    const int cg = j / 16, w = (j % 16) / 4, c = j % 4, part = i / rpt, r = i % rpt, lane = c * 16 + part;
    return (static_cast<int64_t>(vh) * (dv / 16) + cg) * dk * 16 + static_cast<int64_t>(w) * 64 * rpt +
           ((r / vec) * 64 + lane) * vec + r % vec;
}

struct GdnArgs {
    const StepParams *sp;
    const float *proj;     // [M][ld] the projections: q | k | v (conv inputs), then z
    int64_t ld;
    const float *x;        // [M][H] the layer's input rows
    const float *in_norm;
    const uint16_t *ab_w;  // bf16 [2 nv][H]: a rows, then b rows
    const float *A_log, *dt_bias, *conv_w, *gnorm;
    float *c_slots, *s_slots;
    int64_t c_slot_floats, s_slot_floats;
    float *ab;             // [M][2 nv] the a / b dots (written and read in the launch: sc1)
    float *core;           // [M][nv dv] the delta rule's outputs (written and read in the launch: sc1)
    _Float16 *act;         // the output projection's operands
    int64_t act_stride;
    int H, nk, nv, dk, dv, K, conv_dim;
    float eps, qscale;
    int *flags;            // [0, n_ab) the a / b workgroups, [n_ab, n_ab + n_core) the core workgroups
    int *passed;           // the norm workgroups past their waits (the last one clears the flags)
    int *err;
    int n_ab, n_core;      // a / b workgroups (0: the dots given), core workgroups
};

// An a / b workgroup: bf16 rows [4 dg, 4 dg + 4) of in_proj_a | in_proj_b against RMSNorm(x) of a group of rows
// (model.cpp:3548-3551, bf16_rows): the router kernel's rows (layer_common.hpp router_rows), the same bits, stored sc1
__device__ void gdn_ab_role(const GdnArgs &a, int wg, float *lds) {
    trace(GV_K_GDN_CORE, 0);
    // (router_rows<2>: groups of four rows whatever H, its LDS (65 KB at hidden 2048) leaving room for a second
    // workgroup on the CU; for H <= 2048 the same bits as router_rows<1>: the second 8-value group is zeros)
    const int n_dg = (2 * a.nv + kRouterRows - 1) / kRouterRows, dg = wg % n_dg, tg = wg / n_dg;   // (rows, tokens)
    router_rows<2>(dg, tg, 0x7FFF, a.ab_w, 2 * a.nv, a.H, a.x, a.in_norm, a.eps, a.sp, a.ab, true, nullptr, -1, 0, lds);
    trace(GV_K_GDN_CORE, 5);
    signal_done(a.flags + wg);
    trace(GV_K_GDN_CORE, 6);
}

// the sum of a 16-lane row's values on each of its lanes, the same bits on each (pairs, quads, halves, then the row
// by DPP: full-rate VALU, no LDS crossbar round trip)
__device__ inline float row16_sum(float v) {
    v = __fadd_rn(v, dpp_f<0xB1>(v));    // quad_perm [1, 0, 3, 2]
    v = __fadd_rn(v, dpp_f<0x4E>(v));    // quad_perm [2, 3, 0, 1]
    v = __fadd_rn(v, dpp_f<0x141>(v));   // row_half_mirror
    return __fadd_rn(v, dpp_f<0x140>(v));   // row_mirror
}

// the core workgroup's LDS, in floats (M rows, nch channels, K taps)
__host__ __device__ inline size_t gdn_core_lds_floats(int M, int nch, int K) {
    return static_cast<size_t>(2 * M + 2 * K) * nch + (4 + (kMaxConvK - 1)) * kMaxRows;
}

// A core workgroup: value head vh, value columns j0 .. j0 + 15 (wave w: columns j0 + 4 w .. j0 + 4 w + 3, a 16-lane
// row of the wave each); the channels it reads: q and k of the head's key head and its own 16 v columns (three runs of
// the projections' row).
//  1. every load first: the recurrent state of the base slot (registers), the raw conv inputs of every row, the base
//     slot's conv state and the conv weights of those channels (LDS, 16 bytes a load, batched);
//  2. the causal conv (model.cpp:3558-3584), a thread a (row, channel), four at a time: the row's window is its
//     ancestors' raw inputs, newest first, then the base state's; w . window in order, silu; each row's new conv state
//     (its window after it) to its slot, by one workgroup a channel;
//  3. q and k L2-normalised per row (q also by 1 / sqrt(dk)), a wave a (row, q | k);
//  4. the gates from the a / b dots: beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias));
//  5. the delta rule (model.cpp:3614-3666): lane p of a column's 16 holds rows p RPT .. p RPT + RPT - 1 of the state
//     (RPT = dk / 16); per row S *= decay, mem = S^T k, delta = (v - mem) beta, S += k delta^T, o = S^T q (each lane's
//     rows as two interleaved fused multiply-add chains, then the 16 lanes: row16_sum); the row's state to its slot,
//     o to core.
template <int RPT>
__device__ void gdn_core_role(const GdnArgs &a, int w, float *lds) {
    constexpr int VEC = RPT < 4 ? RPT : 4;
    const StepParams *sp = a.sp;
    const int M = sp->M, base = sp->gdn_base, wset = sp->gdn_wset;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dk = a.dk, dv = a.dv, kd = a.nk * dk, ncw = dv / 16, K = a.K;
    const int vh = w / ncw, j0 = (w % ncw) * 16, kh = vh / (a.nv / a.nk), K1 = K - 1;
    const int nch = 2 * dk + 16, n4 = nch / 4;
    float *cv = lds;                    // [M][nch] the raw conv inputs
    float *co = cv + M * nch;           // [M][nch] the conv outputs (q, k then normalised)
    float *bs = co + M * nch;           // [K - 1][nch] the base conv state
    float *cw = bs + K1 * nch;          // [K][nch] the conv weights, tap-major
    float *gd = cw + K * nch;           // [M] decay
    float *gb = gd + kMaxRows;          // [M] beta
    int *par = reinterpret_cast<int *>(gb + kMaxRows);   // [M] each row's parent (-1: the base)
    int *anc = par + kMaxRows;          // [M][K - 1] the n-th newest conv input before the row: a row, or -1 - b for
                                        // the base state's entry b
    uint32_t *vis = reinterpret_cast<uint32_t *>(anc + kMaxRows * (kMaxConvK - 1));   // [M] the rows' visibility masks
    // the channel of local index lc: q of the key head, k of the key head, then the workgroup's v columns
    auto gch = [&](int lc) { return lc < dk ? kh * dk + lc : lc < 2 * dk ? kd + kh * dk + (lc - dk) : 2 * kd + vh * dv + j0 + (lc - 2 * dk); };
    // the delta rule's lanes: column jl = 4 wave + lane / 16 of the workgroup's, rows part RPT .. of it
    const int part = lane & 15, jl = wave * 4 + (lane >> 4), j = j0 + jl;
    const int64_t blk = (static_cast<int64_t>(vh) * ncw + j0 / 16) * dk * 16 + static_cast<int64_t>(wave) * 64 * RPT +
                        lane * VEC;
    float s[RPT];
    auto load = [&](int slot) {
        const float *src = a.s_slots + slot * a.s_slot_floats + blk;
#pragma unroll
        for (int v4 = 0; v4 < RPT / VEC; ++v4) {
            if constexpr (VEC == 4) {
                const float4 v = *reinterpret_cast<const float4 *>(src + v4 * 256);
                s[4 * v4] = v.x, s[4 * v4 + 1] = v.y, s[4 * v4 + 2] = v.z, s[4 * v4 + 3] = v.w;
            } else {
                const float2 v = *reinterpret_cast<const float2 *>(src + v4 * 128);
                s[2 * v4] = v.x, s[2 * v4 + 1] = v.y;
            }
        }
    };
    auto store = [&](int slot) {
        float *dst = a.s_slots + slot * a.s_slot_floats + blk;
#pragma unroll
        for (int v4 = 0; v4 < RPT / VEC; ++v4) {
            if constexpr (VEC == 4)
                *reinterpret_cast<float4 *>(dst + v4 * 256) = make_float4(s[4 * v4], s[4 * v4 + 1], s[4 * v4 + 2], s[4 * v4 + 3]);
            else
                *reinterpret_cast<float2 *>(dst + v4 * 128) = make_float2(s[2 * v4], s[2 * v4 + 1]);
        }
    };
    trace(GV_K_GDN_CORE, 0);
    load(base);
    // the conv weights of the thread's channels (tid, tid + 256, ..: conv_w [ch][K]) and the rows' masks, loaded with
    // the inputs below (one round trip for all; indices clamped, no branch around a load)
    constexpr int kWch = 3;   // channel runs of 256 (nch = 2 dk + 16 <= 768: dk <= 256)
    float wr[kWch][kMaxConvK];
#pragma unroll
    for (int c = 0; c < kWch; ++c) {
        const float *src = a.conv_w + static_cast<int64_t>(gch(min(tid + c * kGdnThreads, nch - 1))) * K;
#pragma unroll
        for (int k = 0; k < kMaxConvK; ++k) wr[c][k] = src[min(k, K - 1)];
    }
    const uint32_t vis_r = sp->vis[min(tid, M - 1)];
    // 1. the raw inputs (rows 0 .. M - 1) and the base conv state (K - 1 rows of conv_dim) in 16-byte pieces: a thread
    // piece c4 of rows r, r + rstep, .. (pieces a row padded to a power of two, so no division), eight loads issued
    // before their LDS stores; then the conv weights, a thread a channel
    {
        const int n4p = 1 << (32 - __clz(n4 - 1)), c4 = tid & (n4p - 1), rstep = kGdnThreads / n4p;
        const int nrows = M + K1;
        if (c4 < n4) {
            const int lc = 4 * c4, gc = gch(lc);
            for (int r0 = tid / n4p; r0 < nrows; r0 += 8 * rstep) {
                float4 r[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {   // (past the end: the last row again, not stored)
                    const int row = min(r0 + u * rstep, nrows - 1);
                    const float *src = row < M ? a.proj + row * a.ld + gc
                                               : a.c_slots + base * a.c_slot_floats + static_cast<int64_t>(row - M) * a.conv_dim + gc;
                    r[u] = *reinterpret_cast<const float4 *>(src);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int row = r0 + u * rstep;
                    if (row < nrows) *reinterpret_cast<float4 *>((row < M ? cv + row * nch : bs + (row - M) * nch) + lc) = r[u];
                }
            }
        }
        if (tid < M) vis[tid] = vis_r;
#pragma unroll
        for (int c = 0; c < kWch; ++c) {   // conv_w [ch][K] to cw [k][lc]
            const int lc = tid + c * kGdnThreads;
            if (lc < nch)
#pragma unroll
                for (int k = 0; k < kMaxConvK; ++k)
                    if (k < K) cw[k * nch + lc] = wr[c][k];
        }
    }
    __syncthreads();
    // the rows' parents (the highest row below each that it sees) and conv windows (the ancestors' inputs, then the
    // base state's newest first), from the masks in LDS
    auto parent = [&](int r) {
        const uint32_t below = r == 0 ? 0u : (vis[r] & ((1u << r) - 1u));
        return below ? 31 - __clz(static_cast<int>(below)) : -1;
    };
    if (tid < M) {
        par[tid] = parent(tid);
        int r = tid, got = 0;
        for (int n = 1; n <= K1; ++n) {
            const int p = r >= 0 ? parent(r) : -1;
            if (p >= 0) ++got;
            anc[tid * (kMaxConvK - 1) + n - 1] = p >= 0 ? p : -1 - (K1 - (n - got));
            r = p;
        }
    }
    __syncthreads();
    trace(GV_K_GDN_CORE, 1);
    // 2. the conv: the q and k channels a thread each (rows split over the threads left: shifts, no division), the 16
    // v channels as (row, column) pairs over every thread; each (row, channel) w . window in order, silu; the conv
    // state's slots written by one workgroup a channel (q and k: the key head's first value head's first workgroup)
    const bool qk_writer = vh % (a.nv / a.nk) == 0 && j0 == 0;
    auto conv_one = [&](int t, int lc) {
        float acc = 0.0f;   // w . window (oldest first: the (K - 1 - k)-th newest before row t), then the input
        for (int k = 0; k < K1; ++k) {
            const int code = anc[t * (kMaxConvK - 1) + (K1 - 1 - k)];
            const float v = code >= 0 ? cv[code * nch + lc] : bs[(-1 - code) * nch + lc];
            acc = __fadd_rn(acc, __fmul_rn(cw[k * nch + lc], v));
        }
        acc = __fadd_rn(acc, __fmul_rn(cw[K1 * nch + lc], cv[t * nch + lc]));
        co[t * nch + lc] = silu_fast(acc);
    };
    // the conv state after row t (its window's newest K - 1 entries, the row's own input last) to its slot: stored
    // after the delta rule, so that no workgroup barrier before then waits for these stores to complete
    auto conv_state_one = [&](int t, int lc) {
        float *dst = a.c_slots + (wset + t) * a.c_slot_floats + gch(lc);
        for (int k = 1; k < K1; ++k) {
            const int code = anc[t * (kMaxConvK - 1) + (K1 - 1 - k)];
            dst[static_cast<int64_t>(k - 1) * a.conv_dim] = code >= 0 ? cv[code * nch + lc] : bs[(-1 - code) * nch + lc];
        }
        dst[static_cast<int64_t>(K1 - 1) * a.conv_dim] = cv[t * nch + lc];
    };
    {
        const int qk = 2 * dk, lg = 31 - __clz(qk);   // (a power of two: 64 .. 512)
        const int per = qk > kGdnThreads ? qk / kGdnThreads : 1;   // channels a thread
        const int t_first = qk >= kGdnThreads ? 0 : tid >> lg, t_step = qk >= kGdnThreads ? 1 : kGdnThreads >> lg;
        for (int c = 0; c < per; ++c) {
            const int lc = qk >= kGdnThreads ? tid + c * kGdnThreads : tid & (qk - 1);
            for (int t0 = t_first; t0 < M; t0 += 4 * t_step) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int t = t0 + u * t_step;
                    if (t < M) conv_one(t, lc);
                }
            }
        }
        for (int p0 = tid; p0 < 16 * M; p0 += 4 * kGdnThreads) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int p = p0 + u * kGdnThreads;
                if (p < 16 * M) conv_one(p >> 4, qk + (p & 15));
            }
        }
    }
    __syncthreads();
    trace(GV_K_GDN_CORE, 2);
    // 3. the L2 norms: pair p = 2 t + (k ? 1 : 0), a wave a pair
    for (int pr = wave; pr < 2 * M; pr += kGdnThreads / 64) {
        float *v = co + (pr >> 1) * nch + (pr & 1) * dk;
        float sq = 0.0f;
        for (int e = lane; e < dk; e += 64) sq = __fadd_rn(sq, __fmul_rn(v[e], v[e]));
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(wave_sum_f(sq), 1e-6f)));
        for (int e = lane; e < dk; e += 64) v[e] = (pr & 1) ? __fmul_rn(v[e], inv) : __fmul_rn(__fmul_rn(v[e], inv), a.qscale);
    }
    // 4. the gates, once the a / b dots are there
    trace(GV_K_GDN_CORE, 3);
    if (a.n_ab) wait_flags(a.flags, a.n_ab, a.err);
    trace(GV_K_GDN_CORE, 4);
    if (tid < M) {
        const int E1 = 2 * a.nv;
        const float av = a.n_ab ? xldf(a.ab, static_cast<uint32_t>(tid * E1 + vh)) : a.ab[tid * E1 + vh];
        const float bv = a.n_ab ? xldf(a.ab, static_cast<uint32_t>(tid * E1 + a.nv + vh)) : a.ab[tid * E1 + a.nv + vh];
        const float x = __fadd_rn(av, a.dt_bias[vh]);
        const float sp_ = x > 20.0f ? x : log1pf(expf(x));
        gd[tid] = expf(-__fmul_rn(expf(a.A_log[vh]), sp_));
        gb[tid] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-bv)));
    }
    __syncthreads();
    // 5. the delta rule
    int held = -1;
    for (int t = 0; t < M; ++t) {
        const int p = par[t];
        if (p != held) load(wset + p);
        const float *row = co + t * nch;
        float q[RPT], k[RPT];
#pragma unroll
        for (int v4 = 0; v4 < RPT / VEC; ++v4) {
            if constexpr (VEC == 4) {
                const float4 qv = *reinterpret_cast<const float4 *>(row + part * RPT + 4 * v4);
                const float4 kv = *reinterpret_cast<const float4 *>(row + dk + part * RPT + 4 * v4);
                q[4 * v4] = qv.x, q[4 * v4 + 1] = qv.y, q[4 * v4 + 2] = qv.z, q[4 * v4 + 3] = qv.w;
                k[4 * v4] = kv.x, k[4 * v4 + 1] = kv.y, k[4 * v4 + 2] = kv.z, k[4 * v4 + 3] = kv.w;
            } else {
                const float2 qv = *reinterpret_cast<const float2 *>(row + part * RPT + 2 * v4);
                const float2 kv = *reinterpret_cast<const float2 *>(row + dk + part * RPT + 2 * v4);
                q[2 * v4] = qv.x, q[2 * v4 + 1] = qv.y;
                k[2 * v4] = kv.x, k[2 * v4 + 1] = kv.y;
            }
        }
        const float v = row[2 * dk + jl], decay = gd[t], beta = gb[t];
        float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
        for (int i = 0; i < RPT; i += 2) {
            s[i] = __fmul_rn(s[i], decay);
            s[i + 1] = __fmul_rn(s[i + 1], decay);
            m0 = fmaf(s[i], k[i], m0);
            m1 = fmaf(s[i + 1], k[i + 1], m1);
        }
        const float delta = __fmul_rn(__fsub_rn(v, row16_sum(__fadd_rn(m0, m1))), beta);
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int i = 0; i < RPT; i += 2) {
            s[i] = fmaf(k[i], delta, s[i]);
            s[i + 1] = fmaf(k[i + 1], delta, s[i + 1]);
            o0 = fmaf(s[i], q[i], o0);
            o1 = fmaf(s[i + 1], q[i + 1], o1);
        }
        const float o = row16_sum(__fadd_rn(o0, o1));
        if (part == 0) xstf(a.core, static_cast<uint32_t>(t * a.nv * dv + vh * dv + j), o);
        store(wset + t);
        held = t;
    }
    trace(GV_K_GDN_CORE, 5);
    signal_done(a.flags + a.n_ab + w);
    trace(GV_K_GDN_CORE, 6);
    // then the conv states (q and k channels: the key head's first workgroup; the 16 v channels: every workgroup),
    // the (row, channel) pairs over the threads: no consumer in this launch waits for them
    const int per_row = qk_writer ? 2 * dk + 16 : 16;
    for (int p = tid; p < per_row * M; p += kGdnThreads) {
        const int t = p / per_row, c = p % per_row;
        conv_state_one(t, qk_writer ? c : 2 * dk + c);
    }
}

// A norm workgroup, row t: once every core workgroup is done, the gated RMSNorm per value head (model.cpp:3670-3682):
// o / rms(o) x w x silu(z) (the head's sum of squares in double over its dv / 8 lanes), then the output projection's
// operands (the int8 path's); the last norm workgroup past its wait clears the launch's flags.
__device__ void gdn_norm_role(const GdnArgs &a, int t) {
    const int M = a.sp->M;
    trace(GV_K_GDN_CORE, 0);
    wait_flags(a.flags + a.n_ab, a.n_core, a.err);
    trace(GV_K_GDN_CORE, 1);
    const int vd = a.nv * a.dv, ng = vd / 8, gph = a.dv / 8, z_off = a.conv_dim;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (q * kGdnThreads >= ng) break;   // uniform
        const int g = threadIdx.x + q * kGdnThreads;
        const bool live = g < ng;
        const int gg = live ? g : 0;
        const float4 p = xld4f(a.core, static_cast<uint32_t>(t * vd + gg * 8)),
                     r = xld4f(a.core, static_cast<uint32_t>(t * vd + gg * 8 + 4));
        float v[8] = {p.x, p.y, p.z, p.w, r.x, r.y, r.z, r.w};
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        for (int off = 1; off < gph; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(static_cast<float>(ss), static_cast<float>(a.dv)), a.eps)));
        const int j0 = (gg % gph) * 8;
        const float *z = a.proj + t * a.ld + z_off + gg * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(__fmul_rn(__fmul_rn(v[i], inv), a.gnorm[j0 + i]), silu_fast(z[i]));
        act16_group(v, g, live, a.act + static_cast<int64_t>(t) * a.act_stride);
    }
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(a.passed, 1) == M - 1;
    __syncthreads();
    if (last) {   // every workgroup has passed its waits: the flags back to zero for the next step
        clear_flags(a.flags, a.n_ab + a.n_core);
        if (threadIdx.x == 0) __hip_atomic_store(a.passed, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The Gated DeltaNet layer after its projections, one launch: workgroups [0, n_ab) the a / b dots of row b (none when
// given), [n_ab, n_ab + n_core) the core, then a norm workgroup a row. Producers have lower ids than their
// consumers (dispatched first, so resident or done when a consumer waits).
template <int RPT>
__global__ __launch_bounds__(kGdnThreads) void gdn_kernel(const GdnArgs a) {
    extern __shared__ float gdn_lds[];
    const int b = blockIdx.x;
    if (b < a.n_ab) gdn_ab_role(a, b, gdn_lds);
    else if (b < a.n_ab + a.n_core) gdn_core_role<RPT>(a, b - a.n_ab, gdn_lds);
    else gdn_norm_role(a, b - a.n_ab - a.n_core);
}

template <int RPT>
int launch_gdn_t(const GdnArgs &a, int M, size_t lds, hipStream_t st) {
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&gdn_kernel<RPT>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(gdn_kernel<RPT>, dim3(static_cast<unsigned>(a.n_ab + a.n_core + M)), dim3(kGdnThreads), lds, st, a);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace

bool gdn_shape_ok(const gv_model_config &c, std::string &why) {
    const int nk = c.gdn_k_heads, nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim, K = c.conv_kernel;
    if (nv == 0) return true;
    if (nk <= 0 || nv < nk || nv % nk != 0) {
        why = "gdn_v_heads must be a positive multiple of gdn_k_heads";
        return false;
    }
    if (dk != 32 && dk != 64 && dk != 128 && dk != 256) {
        why = "gdn_k_dim must be 32, 64, 128 or 256";
        return false;
    }
    if (dv < 16 || dv > 256 || (dv & (dv - 1)) != 0) {
        why = "gdn_v_dim must be a power of two from 16 to 256";
        return false;
    }
    if ((static_cast<int64_t>(nv) * dv) % 128 != 0 || static_cast<int64_t>(nv) * dv > 8192) {
        why = "gdn_v_heads x gdn_v_dim must be a multiple of 128, at most 8192";
        return false;
    }
    if (K < 2 || K > kMaxConvK) {
        why = "conv_kernel must be 2..8";
        return false;
    }
    if (static_cast<int64_t>(2 * nk * dk + nv * dv) > 65536) {
        why = "the Gated DeltaNet's projections are too wide";
        return false;
    }
    if (nv * (dv / 16) + (2 * nv + 3) / 4 * ((c.max_rows + 3) / 4) > kFlagsPerLayer - kGdnFlagBase - 1) {
        why = "too many Gated DeltaNet value heads";
        return false;
    }
    if (c.hidden > 4096) {
        why = "Gated DeltaNet models take hidden up to 4096";
        return false;
    }
    if (gdn_core_lds_floats(c.max_rows, 2 * dk + 16, K) * 4 > 160 * 1024) {
        why = "max_rows x gdn_k_dim too large for the Gated DeltaNet kernel's LDS";
        return false;
    }
    return true;
}

int64_t gdn_conv_dim(const gv_model_config &c) {
    return 2 * static_cast<int64_t>(c.gdn_k_heads) * c.gdn_k_dim + static_cast<int64_t>(c.gdn_v_heads) * c.gdn_v_dim;
}
int64_t gdn_s_floats(const gv_model_config &c) {
    return static_cast<int64_t>(c.gdn_v_heads) * c.gdn_k_dim * c.gdn_v_dim;
}
int64_t gdn_c_floats(const gv_model_config &c) { return gdn_conv_dim(c) * (c.conv_kernel - 1); }

int gdn_launch(Model &m, LayerW &L, int l, int M, bool ab_given, hipStream_t st) {
    const auto &c = m.c;
    GdnArgs a{};
    a.sp = m.sp;
    a.proj = m.qkv_out;
    a.ld = L.qkv.rows;
    a.x = m.x;
    a.in_norm = L.in_norm;
    a.ab_w = L.gdn_ab;
    a.A_log = L.A_log, a.dt_bias = L.dt_bias, a.conv_w = L.conv_w, a.gnorm = L.gnorm;
    a.c_slots = L.c_slots, a.s_slots = L.s_slots;
    a.c_slot_floats = gdn_c_floats(c), a.s_slot_floats = gdn_s_floats(c);
    a.ab = m.rlogits;
    a.core = m.gdn_core;
    a.act = m.act_core;
    a.act_stride = act_halves(static_cast<int64_t>(c.gdn_v_heads) * c.gdn_v_dim);
    a.H = c.hidden, a.nk = c.gdn_k_heads, a.nv = c.gdn_v_heads, a.dk = c.gdn_k_dim, a.dv = c.gdn_v_dim;
    a.K = c.conv_kernel;
    a.conv_dim = static_cast<int>(gdn_conv_dim(c));
    a.eps = c.eps;
    a.qscale = 1.0f / std::sqrt(static_cast<float>(c.gdn_k_dim));
    int *area = m.ctr + static_cast<int64_t>(l) * kFlagsPerLayer;
    a.flags = area + kGdnFlagBase;
    a.passed = area + kFlagsPerLayer - 1;
    a.err = m.err;
    a.n_core = c.gdn_v_heads * (c.gdn_v_dim / 16);
    a.n_ab = ab_given ? 0 : (2 * c.gdn_v_heads + kRouterRows - 1) / kRouterRows * ((M + 3) / 4);   // (router_rows<2>)
    const int nch = 2 * c.gdn_k_dim + 16;
    const size_t core_lds = gdn_core_lds_floats(M, nch, c.conv_kernel) * 4;
    const size_t ab_lds = ab_given ? 0 : static_cast<size_t>(4) * (c.hidden + 8) * 4 + static_cast<size_t>(kRouterRows) * c.hidden * 4;
    const size_t lds = std::max(core_lds, ab_lds);
    switch (c.gdn_k_dim) {   // (rows a lane holds of its column: dk / 16)
    case 32: return launch_gdn_t<2>(a, M, lds, st);
    case 64: return launch_gdn_t<4>(a, M, lds, st);
    case 128: return launch_gdn_t<8>(a, M, lds, st);
    default: return launch_gdn_t<16>(a, M, lds, st);
    }
}

// the states of the layer's base slot from / to host arrays in the reference's layouts (conv [conv_dim][K - 1],
// S [nv][dk][dv])
int gdn_put_state(Model &m, LayerW &L, int slot, const float *conv, const float *S) {
    const auto &c = m.c;
    const int64_t cd = gdn_conv_dim(c), K1 = c.conv_kernel - 1, sn = gdn_s_floats(c);
    if (conv) {
        std::vector<float> d(static_cast<size_t>(cd * K1));
        for (int64_t ch = 0; ch < cd; ++ch)
            for (int64_t k = 0; k < K1; ++k) d[static_cast<size_t>(k * cd + ch)] = conv[ch * K1 + k];
        GV_CHECK_HIP(hipMemcpy(L.c_slots + slot * gdn_c_floats(c), d.data(), d.size() * 4, hipMemcpyHostToDevice));
    }
    if (S) {
        std::vector<float> d(static_cast<size_t>(sn));
        const int nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim;
        for (int vh = 0; vh < nv; ++vh)
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j)
                    d[static_cast<size_t>(s_index(vh, i, j, dk, dv))] = S[(static_cast<int64_t>(vh) * dk + i) * dv + j];
        GV_CHECK_HIP(hipMemcpy(L.s_slots + slot * sn, d.data(), d.size() * 4, hipMemcpyHostToDevice));
    }
    return 0;
}

int gdn_get_state(const Model &m, const LayerW &L, int slot, float *conv, float *S) {
    const auto &c = m.c;
    const int64_t cd = gdn_conv_dim(c), K1 = c.conv_kernel - 1, sn = gdn_s_floats(c);
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    if (conv) {
        std::vector<float> d(static_cast<size_t>(cd * K1));
        GV_CHECK_HIP(hipMemcpy(d.data(), L.c_slots + slot * gdn_c_floats(c), d.size() * 4, hipMemcpyDeviceToHost));
        for (int64_t ch = 0; ch < cd; ++ch)
            for (int64_t k = 0; k < K1; ++k) conv[ch * K1 + k] = d[static_cast<size_t>(k * cd + ch)];
    }
    if (S) {
        std::vector<float> d(static_cast<size_t>(sn));
        GV_CHECK_HIP(hipMemcpy(d.data(), L.s_slots + slot * sn, d.size() * 4, hipMemcpyDeviceToHost));
        const int nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim;
        for (int vh = 0; vh < nv; ++vh)
            for (int i = 0; i < dk; ++i)
                for (int j = 0; j < dv; ++j)
                    S[(static_cast<int64_t>(vh) * dk + i) * dv + j] = d[static_cast<size_t>(s_index(vh, i, j, dk, dv))];
    }
    return 0;
}

GV_ACT_MODE_SETTER(act_mode_set_gdn)

int trace_set_gdn(uint64_t *p) {
    GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &p, sizeof p));
    return 0;
}

}  // namespace gv
