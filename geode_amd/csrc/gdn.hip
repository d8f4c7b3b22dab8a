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

// row t's parent: the highest row below t that it sees (-1 for the first row)
__device__ inline int parent_of(const StepParams *sp, int t) {
    const uint32_t below = t == 0 ? 0u : (sp->vis[t] & ((1u << t) - 1u));
    return below ? 31 - __clz(static_cast<int>(below)) : -1;
}

constexpr int kMaxConvK = 8;
constexpr int kGdnThreads = 256;

// The recurrent state's device layout: value head vh's [dk][dv] in blocks of 16 columns, a block
// [dk / 16 (i4)][4 (part)][16 (column)][4 (e)] for rows i = part (dk / 4) + 4 i4 + e: a lane (part, column) of a
// core wave holds rows part (dk / 4) .. + dk / 4 - 1 of its column, read and written 16 bytes at a time, the wave's
// 64 lanes 1 KB contiguous.
__host__ __device__ inline int64_t s_index(int vh, int i, int j, int dk, int dv) {
    const int rpt = dk / 4, part = i / rpt, ii = i % rpt, i4 = ii / 4, e = ii % 4, cg = j / 16, col = j % 16;
    return (static_cast<int64_t>(vh) * (dv / 16) + cg) * dk * 16 + ((i4 * 4 + part) * 16 + col) * 4 + e;
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
    int n_ab, n_core, cpw; // a / b workgroups (0: the dots given), core workgroups, value columns a core
                           // workgroup takes (min(dv, 64))
};

// An a / b workgroup: the bf16 rows [4 wg, 4 wg + 4) of in_proj_a | in_proj_b against RMSNorm(x) of every row
// (model.cpp:3548-3551, bf16_rows): the router kernel's rows (layer_common.hpp router_rows), the same bits, stored sc1
__device__ void gdn_ab_role(const GdnArgs &a, int wg, float *lds) {
    trace(GV_K_GDN_CORE, 0);
    if (a.H <= 2048) router_rows<1>(wg, a.ab_w, 2 * a.nv, a.H, a.x, a.in_norm, a.eps, a.sp, a.ab, true, nullptr, 0, lds);
    else router_rows<2>(wg, a.ab_w, 2 * a.nv, a.H, a.x, a.in_norm, a.eps, a.sp, a.ab, true, nullptr, 0, lds);
    trace(GV_K_GDN_CORE, 5);
    signal_done(a.flags + wg);
    trace(GV_K_GDN_CORE, 6);
}

// the four parts' partial sums of a lane's column (lanes c, c + 16, c + 32, c + 48) on every lane:
// (p0 + p2) + (p1 + p3), the same bits on each (the additions commute)
__device__ inline float parts_sum(float v) {
    const float s = __fadd_rn(v, __shfl_xor(v, 32, 64));
    return __fadd_rn(s, __shfl_xor(s, 16, 64));
}

// A core workgroup: value head vh, value columns j0 .. j0 + cpw - 1 (a wave each 16 of them); the channels it reads:
// q and k of the head's key head and its own v columns.
//  1. the raw conv inputs of every row and the base slot's conv state for those channels into LDS;
//  2. the causal conv (model.cpp:3558-3584), a thread a channel, the rows from the last to the first (in place: a
//     row's window is its ancestors' raw inputs, newest first, then the base state's): w . window in order, silu;
//     each row's new conv state (its window after it) to its slot, by one workgroup a channel;
//  3. q and k L2-normalised per row (q also by 1 / sqrt(dk)), a wave a (row, q | k);
//  4. the gates from the a / b dots: beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias));
//  5. the delta rule (model.cpp:3614-3666), a wave a 16 columns x 4 parts of dk / 4 rows, the state in registers:
//     per row S *= decay, mem = S^T k, delta = (v - mem) beta, S += k delta^T, o = S^T q (each lane's rows in order,
//     then the parts (p0 + p2) + (p1 + p3)); the row's state to its slot, o to core.
template <int RPT>
__device__ void gdn_core_role(const GdnArgs &a, int w, float *lds) {
    const StepParams *sp = a.sp;
    const int M = sp->M, base = sp->gdn_base, wset = sp->gdn_wset;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dk = a.dk, dv = a.dv, kd = a.nk * dk, ncw = dv / a.cpw;
    const int vh = w / ncw, j0 = (w % ncw) * a.cpw, kh = vh / (a.nv / a.nk), K1 = a.K - 1;
    const int nch = 2 * dk + a.cpw;
    float *cv = lds;                    // [M][nch] raw inputs, then the conv outputs (q, k normalised)
    float *bs = cv + M * nch;           // [K - 1][nch] the base conv state
    float *gd = bs + K1 * nch;          // [M] decay
    float *gb = gd + kMaxRows;          // [M] beta
    int *par = reinterpret_cast<int *>(gb + kMaxRows);   // [M] each row's parent (-1: the base)
    int *anc = par + kMaxRows;          // [M][K - 1] the n-th newest conv input before the row: a row, or -1 - b for
                                        // the base state's entry b
    auto gch = [&](int lc) { return lc < dk ? kh * dk + lc : lc < 2 * dk ? kd + kh * dk + (lc - dk) : 2 * kd + vh * dv + j0 + (lc - 2 * dk); };
    // the delta rule's lanes: wave `wave` takes columns j0 + 16 wave ..; its state prefetched first
    const bool dwave = wave * 16 < a.cpw;
    const int col = lane & 15, part = lane >> 4, jl = wave * 16 + col, j = j0 + jl;
    const int64_t blk = (static_cast<int64_t>(vh) * (dv / 16) + j / 16) * dk * 16 + (part * 16 + col) * 4;
    float s[RPT];
    auto load = [&](int slot) {
        const float *src = a.s_slots + slot * a.s_slot_floats + blk;
#pragma unroll
        for (int i4 = 0; i4 < RPT / 4; ++i4) {
            const float4 v = *reinterpret_cast<const float4 *>(src + i4 * 256);
            s[4 * i4] = v.x, s[4 * i4 + 1] = v.y, s[4 * i4 + 2] = v.z, s[4 * i4 + 3] = v.w;
        }
    };
    trace(GV_K_GDN_CORE, 0);
    if (dwave) load(base);
    if (tid < M) {   // the rows' parents and conv windows (the ancestors' inputs, then the base state's newest first)
        par[tid] = parent_of(sp, tid);
        int r = tid, got = 0;
        for (int n = 1; n <= K1; ++n) {
            const int p = r >= 0 ? parent_of(sp, r) : -1;
            if (p >= 0) ++got;
            anc[tid * (kMaxConvK - 1) + n - 1] = p >= 0 ? p : -1 - (K1 - (n - got));
            r = p;
        }
    }
    // 1. raw inputs and the base conv state
    for (int i = tid; i < M * nch; i += kGdnThreads) {
        const int t = i / nch, lc = i % nch;
        cv[i] = a.proj[t * a.ld + gch(lc)];
    }
    for (int i = tid; i < K1 * nch; i += kGdnThreads) {
        const int k = i / nch, lc = i % nch;
        bs[i] = a.c_slots[base * a.c_slot_floats + static_cast<int64_t>(k) * a.conv_dim + gch(lc)];
    }
    __syncthreads();
    trace(GV_K_GDN_CORE, 1);
    // 2. the conv, a thread a channel; the conv state's slots written by one workgroup a channel (q and k: the key
    // head's first value head's first workgroup)
    const bool qk_writer = vh % (a.nv / a.nk) == 0 && j0 == 0;
    for (int lc = tid; lc < nch; lc += kGdnThreads) {
        const int ch = gch(lc);
        float wc[kMaxConvK];
#pragma unroll
        for (int k = 0; k < kMaxConvK; ++k) wc[k] = k < a.K ? a.conv_w[static_cast<int64_t>(ch) * a.K + k] : 0.0f;
        const bool writer = lc >= 2 * dk || qk_writer;
        for (int t = M - 1; t >= 0; --t) {
            // the window before row t, newest first (its ancestors' raw inputs, still in place: rows below t; then
            // the base state's); win(k) the window oldest first (selects, no indexing)
            float nw[kMaxConvK - 1];
#pragma unroll
            for (int n = 1; n < kMaxConvK; ++n) {
                float v = 0.0f;
                if (n <= K1) {
                    const int code = anc[t * (kMaxConvK - 1) + n - 1];
                    v = code >= 0 ? cv[code * nch + lc] : bs[(-1 - code) * nch + lc];
                }
                nw[n - 1] = v;
            }
            auto win = [&](int k) {
                float v = 0.0f;
#pragma unroll
                for (int m = 0; m < kMaxConvK - 1; ++m)
                    if (m == K1 - 1 - k) v = nw[m];
                return v;
            };
            const float in = cv[t * nch + lc];
            float acc = 0.0f;   // w . window in order, then the row's own input
#pragma unroll
            for (int k = 0; k < kMaxConvK - 1; ++k)
                if (k < K1) acc = __fadd_rn(acc, __fmul_rn(wc[k], win(k)));
            float wl = 0.0f;
#pragma unroll
            for (int k = 0; k < kMaxConvK; ++k)
                if (k == K1) wl = wc[k];
            acc = __fadd_rn(acc, __fmul_rn(wl, in));
            if (writer) {   // the state after the row: the window's last K - 2, then its input
                float *dst = a.c_slots + (wset + t) * a.c_slot_floats + ch;
#pragma unroll
                for (int k = 0; k < kMaxConvK - 1; ++k)
                    if (k < K1) dst[static_cast<int64_t>(k) * a.conv_dim] = k + 1 < K1 ? win(k + 1) : in;
            }
            cv[t * nch + lc] = silu_fast(acc);
        }
    }
    __syncthreads();
    trace(GV_K_GDN_CORE, 2);
    // 3. the L2 norms: pair p = 2 t + (k ? 1 : 0), a wave a pair
    for (int pr = wave; pr < 2 * M; pr += kGdnThreads / 64) {
        float *v = cv + (pr >> 1) * nch + (pr & 1) * dk;
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
    if (dwave) {
        int held = -1;
        for (int t = 0; t < M; ++t) {
            const int p = par[t];
            if (p != held) load(wset + p);
            const float *row = cv + t * nch;
            float q[RPT], k[RPT];
#pragma unroll
            for (int i4 = 0; i4 < RPT / 4; ++i4) {
                const float4 qv = *reinterpret_cast<const float4 *>(row + part * RPT + 4 * i4);
                const float4 kv = *reinterpret_cast<const float4 *>(row + dk + part * RPT + 4 * i4);
                q[4 * i4] = qv.x, q[4 * i4 + 1] = qv.y, q[4 * i4 + 2] = qv.z, q[4 * i4 + 3] = qv.w;
                k[4 * i4] = kv.x, k[4 * i4 + 1] = kv.y, k[4 * i4 + 2] = kv.z, k[4 * i4 + 3] = kv.w;
            }
            const float v = row[2 * dk + jl], decay = gd[t], beta = gb[t];
            float mem = 0.0f;
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                s[i] = __fmul_rn(s[i], decay);
                mem = __fadd_rn(mem, __fmul_rn(s[i], k[i]));
            }
            const float delta = __fmul_rn(__fsub_rn(v, parts_sum(mem)), beta);
            float o = 0.0f;
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                s[i] = __fadd_rn(s[i], __fmul_rn(k[i], delta));
                o = __fadd_rn(o, __fmul_rn(s[i], q[i]));
            }
            o = parts_sum(o);
            if (part == 0) xstf(a.core, static_cast<uint32_t>(t * a.nv * dv + vh * dv + j), o);
            float *dst = a.s_slots + (wset + t) * a.s_slot_floats + blk;
#pragma unroll
            for (int i4 = 0; i4 < RPT / 4; ++i4)
                *reinterpret_cast<float4 *>(dst + i4 * 256) = make_float4(s[4 * i4], s[4 * i4 + 1], s[4 * i4 + 2], s[4 * i4 + 3]);
            held = t;
        }
    }
    trace(GV_K_GDN_CORE, 5);
    signal_done(a.flags + a.n_ab + w);
    trace(GV_K_GDN_CORE, 6);
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
    if (nv * std::max(1, dv / 64) + (2 * nv + 3) / 4 > kFlagsPerLayer - kGdnFlagBase - 1) {
        why = "too many Gated DeltaNet value heads";
        return false;
    }
    if (c.hidden > 4096) {
        why = "Gated DeltaNet models take hidden up to 4096";
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
    a.cpw = std::min(c.gdn_v_dim, 64);
    a.n_core = c.gdn_v_heads * (c.gdn_v_dim / a.cpw);
    a.n_ab = ab_given ? 0 : (2 * c.gdn_v_heads + kRouterRows - 1) / kRouterRows;
    const int nch = 2 * c.gdn_k_dim + a.cpw;
    const size_t core_lds = (static_cast<size_t>(M + c.conv_kernel - 1) * nch + 3 * kMaxRows + kMaxRows * (kMaxConvK - 1)) * 4;
    const size_t ab_lds = ab_given ? 0 : static_cast<size_t>(router_tokens(c.hidden)) * (c.hidden + 8) * 4 +
                                             static_cast<size_t>(kRouterRows) * c.hidden * 4;
    const size_t lds = std::max(core_lds, ab_lds);
    switch (c.gdn_k_dim) {
    case 32: return launch_gdn_t<8>(a, M, lds, st);
    case 64: return launch_gdn_t<16>(a, M, lds, st);
    case 128: return launch_gdn_t<32>(a, M, lds, st);
    default: return launch_gdn_t<64>(a, M, lds, st);
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

int trace_set_gdn(uint64_t *p) {
    GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &p, sizeof p));
    return 0;
}

}  // namespace gv
