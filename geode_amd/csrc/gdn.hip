// gdn.hip - the Gated DeltaNet layer of the verify step (engine/src/model.cpp:3497-3688) on gfx950: the causal
// depthwise conv with silu, the q / k L2 norms and gates, the delta rule on each value head's [dk][dv] state, the
// gated RMSNorm into the output projection's operands. The projections themselves are the step's q4 products
// (in_proj_qkv | in_proj_z as one matrix of two globals, out_proj) and the a / b rows the router kernel's bf16 dots.
//
// States live in slots: two sets of max_rows slots a layer, each slot one row's conv state and recurrent state. A
// verify reads the base slot (the state the last verify or keep left) and writes row t's states into slot t of the
// other set; a row starts from its parent's slot (the tree's), the first row from the base. The states as after any
// row stay until the next verify, so verify_keep (model.cpp:1617-1633: the states as after the last kept row) only
// names a new base slot. Every address a thread writes in a launch is read back by that thread alone, so a launch
// needs no synchronisation between its workgroups.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <vector>

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

// The causal conv, a thread a channel, the rows in order (model.cpp:3558-3584): the parent's last K - 1 inputs
// (oldest first) then the row's own, w . those in order, silu; the row's state (the last K - 1 of them) into its
// slot and the result over the input in proj. Slot layout [K - 1][conv_dim].
__global__ __launch_bounds__(256) void gdn_conv_kernel(const StepParams *__restrict__ sp, float *__restrict__ proj,
                                                       int64_t ld, int conv_dim, int K, const float *__restrict__ w,
                                                       float *__restrict__ slots, int64_t slot_floats) {
    const int ch = blockIdx.x * 256 + threadIdx.x;
    if (ch >= conv_dim) return;
    const int M = sp->M, base = sp->gdn_base, wset = sp->gdn_wset;
    float wc[kMaxConvK], st[kMaxConvK];
#pragma unroll
    for (int k = 0; k < kMaxConvK; ++k) wc[k] = k < K ? w[static_cast<int64_t>(ch) * K + k] : 0.0f;
    auto load = [&](int slot) {
        const float *s = slots + slot * slot_floats + ch;
#pragma unroll
        for (int k = 0; k < kMaxConvK - 1; ++k)
            if (k < K - 1) st[k] = s[static_cast<int64_t>(k) * conv_dim];
    };
    load(base);
    int held = -1;   // the row whose state st holds (-1: the base)
    for (int t = 0; t < M; ++t) {
        const int p = parent_of(sp, t);
        if (p != held) load(wset + p);
        float *x = proj + t * ld + ch;
        const float in = *x;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kMaxConvK - 1; ++k)
            if (k < K - 1) acc = __fadd_rn(acc, __fmul_rn(wc[k], st[k]));
        float wl = 0.0f;
#pragma unroll
        for (int k = 0; k < kMaxConvK; ++k)
            if (k == K - 1) wl = wc[k];
        acc = __fadd_rn(acc, __fmul_rn(wl, in));
#pragma unroll
        for (int k = 0; k < kMaxConvK - 2; ++k)
            if (k + 1 < K - 1) st[k] = st[k + 1];
#pragma unroll
        for (int k = 0; k < kMaxConvK - 1; ++k)
            if (k == K - 2) st[k] = in;
        float *s = slots + (wset + t) * slot_floats + ch;
#pragma unroll
        for (int k = 0; k < kMaxConvK - 1; ++k)
            if (k < K - 1) s[static_cast<int64_t>(k) * conv_dim] = st[k];
        *x = silu_fast(acc);
        held = t;
    }
}

// The recurrent state's device layout: value head vh's [dk][dv] in blocks of 16 columns, a block
// [dk / 16 (i4)][4 (part)][16 (column)][4 (e)] for rows i = part (dk / 4) + 4 i4 + e: a lane (part, column) of the
// core kernel's wave holds rows part (dk / 4) .. + dk / 4 - 1 of its column, read and written 16 bytes at a time, the
// wave's 64 lanes 1 KB contiguous.
__host__ __device__ inline int64_t s_index(int vh, int i, int j, int dk, int dv) {
    const int rpt = dk / 4, part = i / rpt, ii = i % rpt, i4 = ii / 4, e = ii % 4, cg = j / 16, col = j % 16;
    return (static_cast<int64_t>(vh) * (dv / 16) + cg) * dk * 16 + ((i4 * 4 + part) * 16 + col) * 4 + e;
}

struct CoreArgs {
    const StepParams *sp;
    const float *proj;   // [M][ld]: q | k | v after the conv (then z)
    int64_t ld;
    const float *ab;     // [M][2 nv]: a | b (the bf16 rows' dots)
    const float *A_log, *dt_bias;
    float *slots;        // the layer's state slots
    int64_t slot_floats;
    float *core;         // [M][nv dv] the heads' outputs before the gated norm
    int nk, nv, dk, dv;
    float qscale;        // 1 / sqrt(dk), the host's
};

// the four parts' partial sums of a lane's column (lanes c, c + 16, c + 32, c + 48) added in order on every lane
__device__ inline float parts_sum(float v) {
    const int c = threadIdx.x & 15;
    const float p0 = __shfl(v, c, 64), p1 = __shfl(v, c + 16, 64), p2 = __shfl(v, c + 32, 64),
                p3 = __shfl(v, c + 48, 64);
    return __fadd_rn(__fadd_rn(__fadd_rn(p0, p1), p2), p3);
}

// The delta rule (model.cpp:3586-3666), a wave a (value head, 16 columns): per row in order, q and k of the key head
// L2-normalised (q also by 1 / sqrt(dk)), beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias)), then on
// the state S *= decay, mem = S^T k, delta = (v - mem) beta, S += k delta^T, o = S^T q. A lane holds RPT = dk / 4 rows
// of its column in registers: each sum is the part's rows in order, then the four parts in order.
template <int RPT>
__global__ __launch_bounds__(64) void gdn_core_kernel(CoreArgs a) {
    const int ncg = a.dv / 16, vh = blockIdx.x / ncg, cg = blockIdx.x % ncg;
    const int lane = threadIdx.x, col = lane & 15, part = lane >> 4, j = cg * 16 + col;
    const int kh = vh / (a.nv / a.nk), kd = a.nk * a.dk, dk = a.dk;
    const StepParams *sp = a.sp;
    const int M = sp->M, base = sp->gdn_base, wset = sp->gdn_wset;
    const int64_t blk = (static_cast<int64_t>(vh) * ncg + cg) * dk * 16;
    float s[RPT];
    auto load = [&](int slot) {
        const float *src = a.slots + slot * a.slot_floats + blk;
#pragma unroll
        for (int i4 = 0; i4 < RPT / 4; ++i4) {
            const float4 v = *reinterpret_cast<const float4 *>(src + ((i4 * 4 + part) * 16 + col) * 4);
            s[4 * i4] = v.x, s[4 * i4 + 1] = v.y, s[4 * i4 + 2] = v.z, s[4 * i4 + 3] = v.w;
        }
    };
    auto store = [&](int slot) {
        float *dst = a.slots + slot * a.slot_floats + blk;
#pragma unroll
        for (int i4 = 0; i4 < RPT / 4; ++i4)
            *reinterpret_cast<float4 *>(dst + ((i4 * 4 + part) * 16 + col) * 4) =
                make_float4(s[4 * i4], s[4 * i4 + 1], s[4 * i4 + 2], s[4 * i4 + 3]);
    };
    const float A = a.A_log[vh], dtb = a.dt_bias[vh];
    const float eA = expf(A);
    load(base);
    int held = -1;
    for (int t = 0; t < M; ++t) {
        const int p = parent_of(sp, t);
        if (p != held) load(wset + p);
        const float *row = a.proj + t * a.ld;
        float q[RPT], k[RPT];
        const float *qs = row + kh * dk + part * RPT, *ks = row + kd + kh * dk + part * RPT;
#pragma unroll
        for (int i4 = 0; i4 < RPT / 4; ++i4) {
            const float4 qv = *reinterpret_cast<const float4 *>(qs + 4 * i4);
            const float4 kv = *reinterpret_cast<const float4 *>(ks + 4 * i4);
            q[4 * i4] = qv.x, q[4 * i4 + 1] = qv.y, q[4 * i4 + 2] = qv.z, q[4 * i4 + 3] = qv.w;
            k[4 * i4] = kv.x, k[4 * i4 + 1] = kv.y, k[4 * i4 + 2] = kv.z, k[4 * i4 + 3] = kv.w;
        }
        const float v = row[2 * kd + vh * a.dv + j];
        const float av = a.ab[t * 2 * a.nv + vh], bv = a.ab[t * 2 * a.nv + a.nv + vh];
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            sq = __fadd_rn(sq, __fmul_rn(q[i], q[i]));
            sk = __fadd_rn(sk, __fmul_rn(k[i], k[i]));
        }
        const float iq = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(parts_sum(sq), 1e-6f)));
        const float ik = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(parts_sum(sk), 1e-6f)));
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            q[i] = __fmul_rn(__fmul_rn(q[i], iq), a.qscale);
            k[i] = __fmul_rn(k[i], ik);
        }
        const float beta = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-bv)));
        const float x = __fadd_rn(av, dtb);
        const float softplus = x > 20.0f ? x : log1pf(expf(x));
        const float decay = expf(-__fmul_rn(eA, softplus));
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
        if (part == 0) a.core[static_cast<int64_t>(t) * a.nv * a.dv + vh * a.dv + j] = o;
        store(wset + t);
        held = t;
    }
}

// The gated RMSNorm per value head (model.cpp:3670-3682): o / rms(o) x w x silu(z), then the output projection's
// operands (the int8 path's). A workgroup a row; a thread the 8-value groups g, g + 256, ..; a head's groups are
// dv / 8 consecutive lanes, its sum of squares theirs in double.
__global__ __launch_bounds__(256) void gdn_norm_kernel(const StepParams *__restrict__ sp, const float *__restrict__ core,
                                                       const float *__restrict__ proj, int64_t ld, int z_off, int nv,
                                                       int dv, const float *__restrict__ gnorm, float eps,
                                                       _Float16 *__restrict__ act, int64_t act_stride) {
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const int vd = nv * dv, ng = vd / 8, gph = dv / 8;
    const float *o = core + static_cast<int64_t>(t) * vd;
    const float *z = proj + t * ld + z_off;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (q * 256 >= ng) break;   // uniform
        const int g = threadIdx.x + q * 256;
        const bool live = g < ng;
        const int gg = live ? g : 0;
        float v[8];
        {
            const float4 a = *reinterpret_cast<const float4 *>(o + gg * 8), b = *reinterpret_cast<const float4 *>(o + gg * 8 + 4);
            const float tt[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = tt[i];
        }
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += static_cast<double>(v[i]) * static_cast<double>(v[i]);
        for (int off = 1; off < gph; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(static_cast<float>(ss), static_cast<float>(dv)), eps)));
        const int j0 = (gg % gph) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = __fmul_rn(__fmul_rn(__fmul_rn(v[i], inv), gnorm[j0 + i]), silu_fast(z[gg * 8 + i]));
        act16_group(v, g, live, act + static_cast<int64_t>(t) * act_stride);
    }
}

template <int RPT>
int launch_core_t(const CoreArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(gdn_core_kernel<RPT>, dim3(static_cast<unsigned>(a.nv * (a.dv / 16))), dim3(64), 0, st, a);
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
    return true;
}

int64_t gdn_conv_dim(const gv_model_config &c) {
    return 2 * static_cast<int64_t>(c.gdn_k_heads) * c.gdn_k_dim + static_cast<int64_t>(c.gdn_v_heads) * c.gdn_v_dim;
}
int64_t gdn_s_floats(const gv_model_config &c) {
    return static_cast<int64_t>(c.gdn_v_heads) * c.gdn_k_dim * c.gdn_v_dim;
}
int64_t gdn_c_floats(const gv_model_config &c) { return gdn_conv_dim(c) * (c.conv_kernel - 1); }

int gdn_launch(Model &m, LayerW &L, int cls, hipStream_t st) {
    const auto &c = m.c;
    const int64_t conv_dim = gdn_conv_dim(c), ld = L.qkv.rows;
    switch (cls) {
    case GV_K_GDN_CONV:
        hipLaunchKernelGGL(gdn_conv_kernel, dim3(static_cast<unsigned>((conv_dim + 255) / 256)), dim3(256), 0, st, m.sp,
                           m.qkv_out, ld, static_cast<int>(conv_dim), c.conv_kernel, L.conv_w, L.c_slots,
                           gdn_c_floats(c));
        GV_CHECK_HIP(hipGetLastError());
        return 0;
    case GV_K_GDN_CORE: {
        CoreArgs a{};
        a.sp = m.sp;
        a.proj = m.qkv_out;
        a.ld = ld;
        a.ab = m.rlogits;
        a.A_log = L.A_log;
        a.dt_bias = L.dt_bias;
        a.slots = L.s_slots;
        a.slot_floats = gdn_s_floats(c);
        a.core = m.gdn_core;
        a.nk = c.gdn_k_heads, a.nv = c.gdn_v_heads, a.dk = c.gdn_k_dim, a.dv = c.gdn_v_dim;
        a.qscale = 1.0f / std::sqrt(static_cast<float>(c.gdn_k_dim));
        switch (c.gdn_k_dim) {
        case 32: return launch_core_t<8>(a, st);
        case 64: return launch_core_t<16>(a, st);
        case 128: return launch_core_t<32>(a, st);
        default: return launch_core_t<64>(a, st);
        }
    }
    case GV_K_GDN_NORM: {
        const int vd = c.gdn_v_heads * c.gdn_v_dim;
        hipLaunchKernelGGL(gdn_norm_kernel, dim3(static_cast<unsigned>(c.max_rows)), dim3(256), 0, st, m.sp, m.gdn_core,
                           m.qkv_out, ld, static_cast<int>(conv_dim), c.gdn_v_heads, c.gdn_v_dim, L.gnorm, c.eps,
                           m.act_core, act_halves(vd));
        GV_CHECK_HIP(hipGetLastError());
        return 0;
    }
    default: set_error("gdn_launch: not a Gated DeltaNet kernel class"); return -1;
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

}  // namespace gv
