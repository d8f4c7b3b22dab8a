// model.hip - the whole verify step on one MI355X: n <= 32 rows (the last token and its drafts, as a chain or a
// tree) through every layer, the final norm and lm_head, in one host call; the rollback of rejected rows.
//
// Reference: Model::verify_n / verify_keep (engine/src/model.cpp:1483-1634) over forward_batch
// (engine/src/model.cpp:5235-5413); per layer RMSNorm, gated attention (:3690-4019), RMSNorm, the MoE block
// (:4123-4587) and the residual adds; the arithmetic of the int8 path (quantize_activation + matvec_rows_q,
// engine/src/kernels.cpp:1254-1420) with an fp16 KV cache (attend<_Float16>).
//
// Unlike the reference's GPU path (engine/src/gpu8.cpp:798-1081, a host round trip per layer to read the route),
// every expert stays resident in HBM, so routing, the experts and the combine stay on the GPU: one host call.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"
#include "prefill_common.hpp"

namespace gv {

// ---------------------------------------------------------------- kernels
// the rows' embeddings: dequant_row of the embedding matrix (pack.cpp:356-366), bit for bit, to x; then the first
// layer's input RMSNorm and its operands (norm_quant_regs). A workgroup (256 threads) per row.
__global__ __launch_bounds__(256) void embed_kernel(Q4 w, const StepParams *__restrict__ sp, float *__restrict__ x,
                                                    const float *__restrict__ norm_w, float eps,
                                                    _Float16 *__restrict__ act, int64_t act_stride) {
    __shared__ double red[16];
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    float v[4][8];
    dequant_row_regs(w, sp->tokens[t], v, x + static_cast<int64_t>(t) * w.cols);
    norm_quant_regs(v, static_cast<int>(w.cols), norm_w, eps, act + static_cast<int64_t>(t) * act_stride, nullptr, red);
}

// quant_kv_row (model.cpp:3766-3774) of a row held one value a thread (256 threads; threads past the row: live
// false): amax over the row, q = clamp(nearbyint(x * (127 / amax)), -127, 127) to *q (live threads), returns the
// scale amax / 127. Every thread of the workgroup calls it (one barrier).
__device__ inline float kv_quant_row(float x, float *red4, int8_t *q, bool live) {
    const float a = wave_max(live ? fabsf(x) : 0.0f);
    if (threadIdx.x % 64 == 0) red4[threadIdx.x / 64] = a;
    __syncthreads();
    const float amax = fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3]));
    const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    if (live) *q = static_cast<int8_t>(fminf(fmaxf(rintf(__fmul_rn(x, inv)), -127.0f), 127.0f));
    return __fdiv_rn(amax, 127.0f);
}

// Per (row, head): the query heads' and key heads' RMSNorm(1 + w) then partial RoPE on the first rope_dim dims
// (pairs i, i + half; model.cpp:3714-3733, rotary position pos + depth), the keys and values appended to the fp16
// cache at slot pos + row (static_cast<_Float16>: round to nearest even). Query heads go to q_out as two fp16
// arrays [M][nh][hd], hi then lo (hi + lo = the fp32 query to 2^-22), the MFMA operands of the scores.
__global__ __launch_bounds__(256) void qk_rope_kernel(const float *__restrict__ qkv, int64_t ldq, int nh, int nkv, int hd,
                                                      int half, const float *__restrict__ q_norm,
                                                      const float *__restrict__ k_norm, float eps,
                                                      const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                      const StepParams *__restrict__ sp, _Float16 *__restrict__ q_out,
                                                      _Float16 *__restrict__ kv, int8_t *__restrict__ kv8,
                                                      float *__restrict__ kvs, int64_t slots) {
    const int t = blockIdx.x, head = blockIdx.y, i = threadIdx.x;
    if (t >= sp->M) return;
    __shared__ double red[4];
    __shared__ float v[256];
    __shared__ float ared[4];
    const int64_t kv_row = static_cast<int64_t>(nkv) * hd;
    const int slot = sp->pos + t;
    const float *src;
    const float *nw = nullptr;
    int kind, kh = 0;
    if (head < nh) {
        kind = 0;
        src = qkv + t * ldq + static_cast<int64_t>(head) * 2 * hd;
        nw = q_norm;
    } else if (head < nh + nkv) {
        kind = 1;
        kh = head - nh;
        src = qkv + t * ldq + static_cast<int64_t>(nh) * 2 * hd + static_cast<int64_t>(kh) * hd;
        nw = k_norm;
    } else {
        kind = 2;
        kh = head - nh - nkv;
        src = qkv + t * ldq + static_cast<int64_t>(nh) * 2 * hd + kv_row + static_cast<int64_t>(kh) * hd;
    }
    // every load up front, indices clamped (no branch around a load): the value, its norm weight, its rotation
    const float *zero = reinterpret_cast<const float *>(g_zero_act16);
    const int ic = min(i, hd - 1);
    const float xr = src[ic];
    const float nwr = *(nw ? nw + ic : zero);
    const int p = sp->pos + sp->depth[t];
    const int jc = min(i < half ? i : i - half, half - 1);
    const float cr = *(half > 0 ? cos_t + static_cast<int64_t>(p) * half + jc : zero);
    const float sr = *(half > 0 ? sin_t + static_cast<int64_t>(p) * half + jc : zero);
    __builtin_amdgcn_sched_barrier(0);
    const float xv = i < hd ? xr : 0.0f;
    if (kind == 2) {
        if (kv8) {   // quant_kv_row of the value row (model.cpp:3766-3774)
            const float sc = kv_quant_row(xv, ared, kv8 + v_index(slots, hd, nkv, kh, slot, i), i < hd);
            if (i == 0) kvs[kv_scale_index(slots, nkv, 1, kh, slot)] = sc;
        } else if (i < hd) {
            kv[v_index(slots, hd, nkv, kh, slot, i)] = static_cast<_Float16>(xv);
        }
        return;
    }
    double ss = wave_sum(static_cast<double>(xv) * static_cast<double>(xv));
    if (i % 64 == 0) red[i / 64] = ss;
    __syncthreads();
    ss = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(ss / static_cast<double>(hd)), eps)));
    if (i < hd) v[i] = __fmul_rn(__fmul_rn(xv, inv), __fadd_rn(1.0f, nwr));
    __syncthreads();
    if (i >= hd && !(kind == 1 && kv8)) return;   // (the int8 key row's amax takes every thread)
    float out = i < hd ? v[i] : 0.0f;
    if (i < half) out = __fsub_rn(__fmul_rn(v[i], cr), __fmul_rn(v[i + half], sr));
    else if (i < 2 * half) out = __fadd_rn(__fmul_rn(v[i], cr), __fmul_rn(v[i - half], sr));
    if (kind == 0) {   // the query as two halves, hi + lo, for near-fp32 scores from fp16 products
        const int64_t qo = (static_cast<int64_t>(t) * nh + head) * hd + i;
        _Float16 hi, lo;
        split_f16(out, hi, lo);
        q_out[qo] = hi;
        q_out[qo + static_cast<int64_t>(sp->M) * nh * hd] = lo;
    } else if (kv8) {
        const float sc = kv_quant_row(out, ared, kv8 + k_index(slots, hd, kh, slot, i), i < hd);
        if (i == 0) kvs[kv_scale_index(slots, nkv, 0, kh, slot)] = sc;
    } else {
        kv[k_index(slots, hd, kh, slot, i)] = f16_of(out);
    }
}


// Split-KV attention on the matrix cores: a workgroup (4 waves) per (block of 64 positions, KV head), the block's
// keys [64][hd] and values [hd][64] staged in LDS by all its threads (positions past the context as zeros), then a
// wave per 16 queries of the KV head (its query heads x the rows). S^T = K Q^T (v_mfma_f32_16x16x32_f16: fp16 keys,
// the queries as hi + lo fp16 halves, fp32 sums), masked to the context plus each row's visible rows, then per query
// the block's maximum, the weights exp(s - max) and their sum; O^T = V^T P^T with the weights as hi + lo halves.
// Writes the block's partial (weighted values, max, sum) as attend_heads does per block (model.cpp:3894-4018);
// attn_merge joins them.

// NCH = head_dim / 32: every loop over the head's dims, and every load, fixed at compile time (no branch around a
// load, so the compiler waits for exactly the loads each step needs)
// I8: the int8 cache (attend<int8_t>): keys and values staged as fp16 (the int8 values, exact), the block's K and V
// scales in LDS; a score is the dot times (1 / sqrt(hd)) x the position's K scale (model.cpp:3948), the weights'
// sum is the softmax's own and each weight then takes the position's V scale before the values (:3965-3972).
template <int NCH, bool I8>
__global__ __launch_bounds__(256) void attn_block_kernel(const _Float16 *__restrict__ q16,
                                                         const void *__restrict__ kvp,
                                                         const float *__restrict__ kvs, int64_t slots, int nh,
                                                         int nkv, const StepParams *__restrict__ sp,
                                                         float *__restrict__ parts, int nb_max) {
    constexpr int hd = NCH * 32;
    extern __shared__ _Float16 lds_h[];
    __shared__ float sc_l[I8 ? 256 : 1];   // int8: the block's K scales [0, 64), V scales [64, 128)
    trace(GV_K_ATTN, 0);
    const int pos = sp->pos, M = sp->M, total = pos + M;
    // workgroup i -> (block, KV head): the context's last block (usually a few new rows) of every KV head takes the
    // highest ids, so that the workgroups past one a CU, dispatched last, are those short ones
    const int nb_live = (total + kAttnBlock - 1) / kAttnBlock, wi = blockIdx.x;
    if (wi >= nb_live * nkv) return;
    const int b = wi < (nb_live - 1) * nkv ? wi / nkv : nb_live - 1;
    const int kh = wi < (nb_live - 1) * nkv ? wi % nkv : wi - (nb_live - 1) * nkv;
    const int s0 = b * kAttnBlock;
    const int live = total - s0;   // positions of the block inside the context (1 .. 64)
    const int kld = attn_k_ld(hd);
    _Float16 *ks = lds_h, *vs = lds_h + kAttnBlock * kld;
    const int group = nh / nkv, NQ = group * M, nqt = (NQ + 15) / 16;
    const int wave = threadIdx.x / 64, l = threadIdx.x % 64, lq = l % 16, lg = l / 16;
    const int64_t qlo = static_cast<int64_t>(M) * nh * hd;
    // the queries of tile qt as B operands (hi and lo halves): dims ch * 32 + 8 lg .. + 8 of query qt * 16 + lq
    auto load_q = [&](int qt, half8 (&qb)[NCH], half8 (&ql)[NCH]) {
        // (a query past the tile's end reads query 0: its scores are masked and its output is not written, so
        // nothing waits on a select of the loaded values)
        const int qi = qt * 16 + lq;
        const bool ok = qi < NQ;
        const int tq = ok ? qi / group : 0, hq = kh * group + (ok ? qi % group : 0);
        const _Float16 *qp = q16 + (static_cast<int64_t>(tq) * nh + hq) * hd + 8 * lg;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            qb[ch] = *reinterpret_cast<const half8 *>(qp + ch * 32);
            ql[ch] = *reinterpret_cast<const half8 *>(qp + qlo + ch * 32);
        }
    };
    half8 qb[NCH], ql[NCH];
    load_q(wave, qb, ql);   // the wave's first tile of queries, in flight with the staging loads
    // the visibility masks of the lane's query rows (sp->vis: bit j = the row sees new row j), loaded with them
    auto vis_of = [&](int qt) { return sp->vis[min((qt * 16 + lq) / group, M - 1)]; };
    uint32_t vis_first = vis_of(wave);
    if constexpr (I8) {   // int8: a block's K (or V) is 64 x hd bytes, 16 a load; fp16 in the LDS
        const int8_t *kv8 = static_cast<const int8_t *>(kvp);
        const int8_t *kg = kv8 + k_index(slots, hd, kh, s0, 0);
        const int8_t *vg = kv8 + v_index(slots, hd, nkv, kh, s0, 0);
        constexpr int nld = kAttnBlock * hd / 16, nl = (nld + 255) / 256;   // 16-byte loads of each, a thread's
        uint4 kr[nl], vr[nl];
#pragma unroll
        for (int u = 0; u < nl; ++u) {
            const int i = min(static_cast<int>(threadIdx.x) + u * 256, nld - 1);
            // (rows past the context read the last live row again, from the cache: their scores are masked and
            // their weights zero)
            const int kr_row = min(i / (hd / 16), live - 1);
            kr[u] = *reinterpret_cast<const uint4 *>(kg + static_cast<int64_t>(kr_row) * hd + (i % (hd / 16)) * 16);
            const int vd = i / (kAttnBlock / 16), vc = min(i % (kAttnBlock / 16), (live - 1) / 16);
            vr[u] = *reinterpret_cast<const uint4 *>(vg + (static_cast<int64_t>(vd) * (kAttnBlock / 16) + vc) * 16);
        }
        // the block's scales: thread j < 64 the K scale of position j, 64 <= j < 128 the V scale (0 past the
        // context, so that a weight 0 stays 0)
        const int j = threadIdx.x % kAttnBlock, which = (threadIdx.x / kAttnBlock) & 1;
        const float scv = kvs[kv_scale_index(slots, nkv, which, kh, s0 + j)];
        __builtin_amdgcn_sched_barrier(0);
        auto to_h8 = [](uint32_t lo, uint32_t hi) {   // 8 int8 values (little-endian) as fp16 (exact)
            half8 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[e] = static_cast<_Float16>(static_cast<int8_t>((lo >> (8 * e)) & 0xFF));
                h[4 + e] = static_cast<_Float16>(static_cast<int8_t>((hi >> (8 * e)) & 0xFF));
            }
            return h;
        };
#pragma unroll
        for (int u = 0; u < nl; ++u) {   // (a thread past nld stores item nld - 1 again: no branch to sink loads into)
            const int i = min(static_cast<int>(threadIdx.x) + u * 256, nld - 1);
            const int r = i / (hd / 16), c = i % (hd / 16);
            *reinterpret_cast<half8 *>(ks + r * kld + c * 16) = to_h8(kr[u].x, kr[u].y);
            *reinterpret_cast<half8 *>(ks + r * kld + c * 16 + 8) = to_h8(kr[u].z, kr[u].w);
            const int d = i / (kAttnBlock / 16), cv = i % (kAttnBlock / 16);
            *reinterpret_cast<half8 *>(vs + d * kAttnVld + cv * 16) = to_h8(vr[u].x, vr[u].y);
            *reinterpret_cast<half8 *>(vs + d * kAttnVld + cv * 16 + 8) = to_h8(vr[u].z, vr[u].w);
        }
        sc_l[threadIdx.x] = which == 1 && s0 + j >= total ? 0.0f : scv;   // (threads >= 128: copies, unused)
    } else {   // stage: keys row by row, values (already [hd][64] in the cache) row by row; 8 halves a load, every
               // load of the thread issued before the first store (NCH of each)
        const _Float16 *kv = static_cast<const _Float16 *>(kvp);
        const _Float16 *kg = kv + k_index(slots, hd, kh, s0, 0);
        const _Float16 *vg = kv + v_index(slots, hd, nkv, kh, s0, 0);
        const int kpr = hd / 8;   // loads a key row
        const int nl = hd / 32;   // loads a thread of each
        uint4 kr[8], vr[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (u >= nl) break;
            const int i = threadIdx.x + u * 256;
            const int r = i / kpr, c = i % kpr;
            // (rows past the context read the last live row again, from the cache: their scores are masked; values
            // past it are zeroed below, as a weight 0 times a stale non-finite value would not be 0, and their
            // 8-position pieces past the last live one read that one again)
            kr[u] = *reinterpret_cast<const uint4 *>(kg + static_cast<int64_t>(min(r, live - 1)) * hd + c * 8);
            const int vd = i / (kAttnBlock / 8), vc = min(i % (kAttnBlock / 8), (live - 1) / 8);
            vr[u] = *reinterpret_cast<const uint4 *>(vg + (static_cast<int64_t>(vd) * (kAttnBlock / 8) + vc) * 8);
        }
        __builtin_amdgcn_sched_barrier(0);   // every load issued before the first store waits for one
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (u >= nl) break;
            const int i = threadIdx.x + u * 256;
            const int r = i / kpr, c = i % kpr;
            *reinterpret_cast<uint4 *>(ks + r * kld + c * 8) = kr[u];
            const int d = i / (kAttnBlock / 8), cv = i % (kAttnBlock / 8);
            const int lim = total - s0 - cv * 8;   // positions of this load inside the context
            auto keep = [&](int k) {   // the word's halves (positions 2k, 2k + 1) inside the context: kept (no branch)
                return lim >= 2 * k + 2 ? 0xFFFFFFFFu : lim == 2 * k + 1 ? 0xFFFFu : 0u;
            };
            const uint4 v = make_uint4(vr[u].x & keep(0), vr[u].y & keep(1), vr[u].z & keep(2), vr[u].w & keep(3));
            *reinterpret_cast<uint4 *>(vs + d * kAttnVld + cv * 8) = v;
        }
    }
    __syncthreads();
    trace(GV_K_ATTN, 1);
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(hd)));
    for (int qt = wave; qt < nqt; qt += 4) {
        if (qt != wave) load_q(qt, qb, ql);
        const int qi = qt * 16 + lq;
        const bool qvalid = qi < NQ;
        const int tq = qvalid ? qi / group : 0, hq = kh * group + (qvalid ? qi % group : 0);
        const uint32_t vis = qvalid ? (qt == wave ? vis_first : vis_of(qt)) : 0u;
        // the four 16-position tiles' scores, hi and lo products apart: eight independent MFMA chains. The keys'
        // operands come from LDS a group of KG chunks at a time, the next group's reads issued before the current
        // group's products (double-buffered), so that no product waits for a read issued just before it
        constexpr int KG = 2, NKG = (NCH + KG - 1) / KG;
        float4v ch_[4], cl_[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) ch_[pt] = cl_[pt] = float4v{0, 0, 0, 0};
        half8 kb[2][KG][4];
        auto load_k = [&](int g, half8 (&dst)[KG][4]) {
#pragma unroll
            for (int c = 0; c < KG; ++c)
#pragma unroll
                for (int pt = 0; pt < 4; ++pt)
                    if (g * KG + c < NCH)   // (compile time: the loops are unrolled)
                        dst[c][pt] = *reinterpret_cast<const half8 *>(ks + (pt * 16 + lq) * kld + 8 * lg + (g * KG + c) * 32);
        };
        load_k(0, kb[0]);
#pragma unroll
        for (int g = 0; g < NKG; ++g) {
            if (g + 1 < NKG) load_k(g + 1, kb[(g + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = 0; c < KG; ++c)
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    const int ch = g * KG + c;
                    if (ch >= NCH) break;
                    ch_[pt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[g & 1][c][pt], qb[ch], ch_[pt], 0, 0, 0);
                    cl_[pt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[g & 1][c][pt], ql[ch], cl_[pt], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        float sc[4][4];
        float mx = -__builtin_inff();
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {   // S^T[position pt*16 + 4 lg + r][query lq]
                const int slot = s0 + pt * 16 + 4 * lg + r;
                const bool ok = qvalid && slot < total && (slot < pos || ((vis >> (slot - pos)) & 1u));
                const float f = I8 ? scale * sc_l[pt * 16 + 4 * lg + r] : scale;
                sc[pt][r] = ok ? (ch_[pt][r] + cl_[pt][r]) * f : -__builtin_inff();
                mx = fmaxf(mx, sc[pt][r]);
            }
        if (qt == wave) trace(GV_K_ATTN, 2);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float lsum = 0.0f;
        half4 pe[4], pl[4];   // the weights as hi + lo halves
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = sc[pt][r] == -__builtin_inff() ? 0.0f : expf(sc[pt][r] - mx);
                _Float16 eh, el;
                split_f16(I8 ? e * sc_l[kAttnBlock + pt * 16 + 4 * lg + r] : e, eh, el);
                pe[pt][r] = eh;
                pl[pt][r] = el;
                lsum += e;
            }
        lsum += __shfl_xor(lsum, 16, 64);
        lsum += __shfl_xor(lsum, 32, 64);
        // P^T operands of the two 32-position chunks: k-slot j < 4 is position 32 kc + 4 lg + j, j >= 4 is
        // 32 kc + 16 + 4 lg + j - 4; the V^T operands take the same positions
        half8 pb[2], pbl[2];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pb[kc][j] = pe[2 * kc][j];
                pb[kc][4 + j] = pe[2 * kc + 1][j];
                pbl[kc][j] = pl[2 * kc][j];
                pbl[kc][4 + j] = pl[2 * kc + 1][j];
            }
        float *dst = parts + ((static_cast<int64_t>(tq) * nh + hq) * nb_max + b) * (hd + 2);
        constexpr int NDT = hd / 16;   // 16-dim tiles of the head (2 NCH: not always a multiple of four)
        constexpr int NVG = (NDT + 3) / 4;
        // the values' operands of four 16-dim tiles (both 32-position chunks), read a group ahead like the keys'
        half8 vb[2][2][4];
        auto load_v = [&](int vg, half8 (&dstv)[2][4]) {
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (4 * vg + k < NDT) {   // (compile time)
                        const _Float16 *vrow = vs + ((4 * vg + k) * 16 + lq) * kAttnVld;
                        const half4 lo = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 4 * lg);
                        const half4 hi = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 16 + 4 * lg);
                        dstv[kc][k] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    }
        };
        load_v(0, vb[0]);
#pragma unroll
        for (int vg = 0; vg < NVG; ++vg) {   // four 16-dim tiles at a time, hi and lo apart
            const int dt0 = 4 * vg;
            if (vg + 1 < NVG) load_v(vg + 1, vb[(vg + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            float4v oh[4], ol[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) oh[k] = ol[k] = float4v{0, 0, 0, 0};
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (dt0 + k >= NDT) break;   // (compile time: the loops are unrolled)
                    oh[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb[vg & 1][kc][k], pb[kc], oh[k], 0, 0, 0);
                    ol[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb[vg & 1][kc][k], pbl[kc], ol[k], 0, 0, 0);
                }
            // O^T[dim dt*16 + 4 lg + r][query lq]
            if (qvalid)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (dt0 + k >= NDT) break;
                    const float4v c = oh[k] + ol[k];
                    *reinterpret_cast<float4 *>(dst + (dt0 + k) * 16 + 4 * lg) = make_float4(c[0], c[1], c[2], c[3]);
                }
        }
        if (qvalid && lg == 0) {
            dst[hd] = mx;
            dst[hd + 1] = lsum;
        }
        if (qt == wave) trace(GV_K_ATTN, 3);
    }
}

// The blocks joined per (row, head): exp(block max - max), the sums, 1 / sum, times sigmoid(gate)
// (model.cpp:3830-3855), then the row's operands for the output projection (the int8 path, act16 layout). A
// workgroup (4 waves) per (row, head): the blocks' weights once, then wave w adds the blocks b = w mod 4, four dims
// a lane, and the waves' sums are added in order.
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ parts, const float *__restrict__ qkv,
                                                         int64_t ldq, int nh, int hd, int nb_max,
                                                         const StepParams *__restrict__ sp,
                                                         _Float16 *__restrict__ act, int64_t act_stride) {
    __shared__ float fw[1024];
    __shared__ float red[2][4];
    __shared__ float4 osum[4][64];
    trace(GV_K_MERGE, 0);
    const int t = blockIdx.x, h = blockIdx.y;
    if (t >= sp->M) return;
    const int nbw = (sp->pos + sp->M + kAttnBlock - 1) / kAttnBlock;
    const int ld = hd + 2;
    const float *base = parts + ((static_cast<int64_t>(t) * nh + h) * nb_max) * ld;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Every load of the first pass issued at once: the blocks' maxima and sums (four blocks a thread), the first
    // kMergeBatch blocks' values of the wave (blocks wave, wave + 4, ...; four dims a lane) and the gate values of
    // wave 0's output dims; the values do not wait for the maximum (their weights are applied after).
    constexpr int kMergeBatch = 36;   // blocks a wave (144 blocks a workgroup: 9216 positions)
    // Unconditional loads, indices clamped: a block past nbw reads block nbw - 1 again (its maximum changes no
    // maximum; its sum and values are never added, their weights being 0), a lane past the head's dims reads the
    // last four (unused).
    float bm[4], bs[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int bb = min(static_cast<int>(threadIdx.x) + 256 * k, nbw - 1);
        bm[k] = base[bb * ld + hd];
        bs[k] = base[bb * ld + hd + 1];
    }
    const bool dl = lane * 4 < hd;
    const int dc = min(lane * 4, hd - 4);
    float4 pv[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
        pv[u] = *reinterpret_cast<const float4 *>(base + min(wave + 4 * u, nbw - 1) * ld + dc);
    const int ng = hd / 8;
    float gate[8];
    {
        const float *gp = qkv + t * ldq + static_cast<int64_t>(h) * 2 * hd + hd + 8 * min(lane, ng - 1);
        const float4 a = *reinterpret_cast<const float4 *>(gp), b = *reinterpret_cast<const float4 *>(gp + 4);
        const float g8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) gate[i] = g8[i];
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before the first use waits for one
    float mx = fmaxf(fmaxf(bm[0], bm[1]), fmaxf(bm[2], bm[3]));
    mx = wave_max(mx);
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    trace(GV_K_MERGE, 1);
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int bb = threadIdx.x + 256 * k;
        if (bb >= nbw) break;
        const float f = bm[k] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(bm[k], mx));
        fw[bb] = f;
        l = __builtin_fmaf(bs[k], f, l);
    }
    l = static_cast<float>(wave_sum(static_cast<double>(l)));
    if (lane == 0) red[1][wave] = l;
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3]);
    // wave w: blocks w, w + 4, ... in order; lane: dims 4 lane .. 4 lane + 3 (hd / 4 lanes)
    float4 o = make_float4(0, 0, 0, 0);
    if (dl) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const int bb = wave + 4 * u;
            const float f = bb < nbw ? fw[bb] : 0.0f;   // (a clamped block: weight 0)
            o.x = __builtin_fmaf(pv[u].x, f, o.x);
            o.y = __builtin_fmaf(pv[u].y, f, o.y);
            o.z = __builtin_fmaf(pv[u].z, f, o.z);
            o.w = __builtin_fmaf(pv[u].w, f, o.w);
        }
        for (int b = wave + 4 * kMergeBatch; b < nbw; b += 64) {   // longer contexts: sixteen blocks at a time
            float4 w4[16];
            float f[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const bool in = b + 4 * u < nbw;
                w4[u] = in ? *reinterpret_cast<const float4 *>(base + (b + 4 * u) * ld + lane * 4) : make_float4(0, 0, 0, 0);
                f[u] = in ? fw[b + 4 * u] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                o.x = __builtin_fmaf(w4[u].x, f[u], o.x);
                o.y = __builtin_fmaf(w4[u].y, f[u], o.y);
                o.z = __builtin_fmaf(w4[u].z, f[u], o.z);
                o.w = __builtin_fmaf(w4[u].w, f[u], o.w);
            }
        }
    }
    osum[wave][lane] = o;
    __syncthreads();
    trace(GV_K_MERGE, 2);
    // the gated output, 8 dims (one k-group of the projection's operands) a lane of wave 0
    if (wave == 0) {
        const int g = lane;
        const bool live = g < ng;
        float v[8];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int li = live ? 2 * g + half : 0;
            float4 s4 = osum[0][li];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const float4 a = osum[w][li];
                s4.x += a.x, s4.y += a.y, s4.z += a.z, s4.w += a.w;
            }
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gate[4 * half + i])));
                v[4 * half + i] = __fmul_rn(__fmul_rn(sv[i], inv), sig);
            }
        }
        act16_group(v, h * ng + g, live, act + static_cast<int64_t>(t) * act_stride);
    }
    trace(GV_K_MERGE, 3);
}

// attn_merge_kernel's arithmetic with the head's dims split over workgroups (head_dim a multiple of 64): a workgroup
// per (row, head, 64 dims), four times the workgroups with a quarter of the loads each at head_dim 256. Lane
// (phase ph = 4 wave + lane / 16, dims 4 (lane % 16) .. + 3 of the part) adds the blocks b = ph mod 16 in order; the
// sixteen phases' sums are then added in a fixed order (lanes by xor 16 then 32, the waves in order).
__global__ __launch_bounds__(256) void attn_merge64_kernel(const float *__restrict__ parts, const float *__restrict__ qkv,
                                                           int64_t ldq, int nh, int hd, int nb_max,
                                                           const StepParams *__restrict__ sp,
                                                           _Float16 *__restrict__ act, int64_t act_stride) {
    __shared__ float fw[1024];
    __shared__ float red[2][4];
    __shared__ float4 osum[4][16];
    trace(GV_K_MERGE, 0);
    const int t = blockIdx.x, h = blockIdx.y, part = blockIdx.z;
    if (t >= sp->M) return;
    const int nbw = (sp->pos + sp->M + kAttnBlock - 1) / kAttnBlock;
    const int ld = hd + 2;
    const float *base = parts + ((static_cast<int64_t>(t) * nh + h) * nb_max) * ld;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ph = 4 * wave + lane / 16, dq = lane % 16;
    const int d0 = part * 64 + 4 * dq;
    // every load of the first pass at once (indices clamped as in attn_merge_kernel): the blocks' maxima and sums,
    // the phase's first kB blocks' four dims, the gate values of wave 0's groups
    float bm[4], bs[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int bb = min(static_cast<int>(threadIdx.x) + 256 * k, nbw - 1);
        bm[k] = base[bb * ld + hd];
        bs[k] = base[bb * ld + hd + 1];
    }
    constexpr int kB = 9;   // blocks a phase (144 blocks a workgroup: 9216 positions)
    float4 pv[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) pv[u] = *reinterpret_cast<const float4 *>(base + min(ph + 16 * u, nbw - 1) * ld + d0);
    const int g = min(lane, 7);   // wave 0: lane g < 8 takes group part * 8 + g (8 dims)
    float gate[8];
    {
        const float *gp = qkv + t * ldq + static_cast<int64_t>(h) * 2 * hd + hd + part * 64 + 8 * g;
        const float4 a = *reinterpret_cast<const float4 *>(gp), b = *reinterpret_cast<const float4 *>(gp + 4);
        const float g8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) gate[i] = g8[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    float mx = fmaxf(fmaxf(bm[0], bm[1]), fmaxf(bm[2], bm[3]));
    mx = wave_max(mx);
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    trace(GV_K_MERGE, 1);
    mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int bb = threadIdx.x + 256 * k;
        if (bb >= nbw) break;
        const float f = bm[k] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(bm[k], mx));
        fw[bb] = f;
        l = __builtin_fmaf(bs[k], f, l);
    }
    l = static_cast<float>(wave_sum(static_cast<double>(l)));
    if (lane == 0) red[1][wave] = l;
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3]);
    float4 o = make_float4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < kB; ++u) {
        const int bb = ph + 16 * u;
        const float f = bb < nbw ? fw[bb] : 0.0f;   // (a clamped block: weight 0)
        o.x = __builtin_fmaf(pv[u].x, f, o.x);
        o.y = __builtin_fmaf(pv[u].y, f, o.y);
        o.z = __builtin_fmaf(pv[u].z, f, o.z);
        o.w = __builtin_fmaf(pv[u].w, f, o.w);
    }
    for (int b = ph + 16 * kB; b < nbw; b += 16 * 8) {   // longer contexts: eight blocks a phase at a time
        float4 w4[8];
        float f[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const bool in = b + 16 * u < nbw;
            w4[u] = in ? *reinterpret_cast<const float4 *>(base + (b + 16 * u) * ld + d0) : make_float4(0, 0, 0, 0);
            f[u] = in ? fw[b + 16 * u] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            o.x = __builtin_fmaf(w4[u].x, f[u], o.x);
            o.y = __builtin_fmaf(w4[u].y, f[u], o.y);
            o.z = __builtin_fmaf(w4[u].z, f[u], o.z);
            o.w = __builtin_fmaf(w4[u].w, f[u], o.w);
        }
    }
#pragma unroll
    for (int x = 16; x <= 32; x *= 2) {   // the wave's four phases: (p0 + p1) + (p2 + p3) on every lane
        o.x += __shfl_xor(o.x, x, 64);
        o.y += __shfl_xor(o.y, x, 64);
        o.z += __shfl_xor(o.z, x, 64);
        o.w += __shfl_xor(o.w, x, 64);
    }
    if (lane < 16) osum[wave][lane] = o;
    __syncthreads();
    trace(GV_K_MERGE, 2);
    if (wave == 0) {   // the gated output of the part's 8 groups (a k-group of the projection's operands a lane)
        float v[8];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float4 s4 = osum[0][2 * g + half];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const float4 a = osum[w][2 * g + half];
                s4.x += a.x, s4.y += a.y, s4.z += a.z, s4.w += a.w;
            }
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gate[4 * half + i])));
                v[4 * half + i] = __fmul_rn(__fmul_rn(sv[i], inv), sig);
            }
        }
        act16_group(v, h * (hd / 8) + part * 8 + g, lane < 8, act + static_cast<int64_t>(t) * act_stride);
    }
    trace(GV_K_MERGE, 3);
}

// the route alone (rows' logits given after the router: the MoE block entry point)
__global__ __launch_bounds__(1024) void route_kernel(const float *__restrict__ logits, int E, int K,
                                                    const StepParams *__restrict__ sp, RouteState *__restrict__ rs,
                                                    int32_t *__restrict__ ids_out) {
    __shared__ int ids[kMaxRows * 16];
    __shared__ int cnt[257], start[257], slot_of[257];
    __shared__ unsigned rows[257];
    __shared__ int wtot[2][16];
    route_all(logits, E, K, sp->M, rs, ids_out, RouteLds{ids, cnt, start, slot_of, rows, wtot});
}

template <int GPT>   // 8-value groups a thread takes per row: 1 for H <= 2048, 2 up to 4096
__global__ __launch_bounds__(256) void router_kernel(const uint16_t *__restrict__ w, int E1, int H,
                                                     const float *__restrict__ x, const float *__restrict__ norm_w,
                                                     float eps, const StepParams *__restrict__ sp,
                                                     float *__restrict__ logits, _Float16 *__restrict__ act,
                                                     int64_t act_stride, int route, int E, int K,
                                                     RouteState *__restrict__ rs, int32_t *__restrict__ ids_out,
                                                     int *__restrict__ counter, int n_dg, int shared_dg) {
    // workgroup b: router rows 4 (b % n_dg) .., token group b / n_dg; it writes the experts' operands of row
    // (b / n_dg) TG + b % n_dg (when b % n_dg < TG: every row's by one workgroup, n_dg >= min(M, TG)).
    // shared_dg >= 0 (the routed logits given): the last row group of each token group is shared_dg instead, the one
    // holding the shared expert's gate row; the others then only make the operands (and logits that are replaced)
    extern __shared__ float lds_f[];
    constexpr int TG = GPT == 1 ? 8 : 4;
    const int dg0 = static_cast<int>(blockIdx.x) % n_dg, tg = static_cast<int>(blockIdx.x) / n_dg;
    const int dg = shared_dg >= 0 && dg0 == n_dg - 1 ? shared_dg : dg0;
    router_rows<GPT>(dg, tg, 0x7FFF, w, E1, H, x, norm_w, eps, sp, logits, false, act, dg < TG ? tg * TG + dg : -1,
                     act_stride, lds_f);
    if (!route) return;
    // the last workgroup to finish routes the rows (the others' logits made visible by their fences)
    __shared__ int s_last;
    __shared__ int wtot[2][16];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(counter, 1) == static_cast<int>(gridDim.x) - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (threadIdx.x == 0) *counter = 0;   // ready for the next launch
    int *ids = reinterpret_cast<int *>(lds_f);
    int *cnt = ids + kMaxRows * 16, *start = cnt + 260, *slot_of = start + 260;
    unsigned *rows = reinterpret_cast<unsigned *>(slot_of + 260);
    route_all(logits, E, K, sp->M, rs, ids_out, RouteLds{ids, cnt, start, slot_of, rows, wtot});
}

// ---------------------------------------------------------------- output projection, router and route in one launch
// Three roles of one launch, each consuming the previous one's results as soon as they exist (no kernel boundary, no
// cache maintenance: common.hpp's sc1 exchange and counters):
//   workgroups [0, n_o)            the output projection x += O core (gemv_q4_kernel's products), x stored sc1;
//   workgroups [n_o, n_o + n_r)    the router: each loads its 4 router rows and the post-norm weights first, then
//                                  waits for the projection, loads the rows of x, makes the post-attention RMSNorm
//                                  and the router logits (router_kernel's arithmetic), logits stored sc1;
//   workgroup n_o + n_r            the route (route_kernel's): waits for the router, then routes the rows.
// Workgroups are dispatched in id order, so each waits only for workgroups that are resident or done. The route's
// workgroup clears the launch's flags once everything has passed them (for the next step).
constexpr int kRT = 260;   // floats a transposed router chain (256 steps + 4: the lanes' 16-byte reads spread over banks)
constexpr int kMaxRowsMixOut = 8;   // rows the fused launch takes (the verify step's chains; more rows: the kernels apart)

struct MixOutArgs {
    Q4 o;                       // the output projection [H x nh hd]
    const _Float16 *act_core;   // its operands (act16 rows)
    int64_t core_stride;
    float *x;                   // the residual rows [M][H]
    int o_per;                  // row tiles a projection workgroup takes
    const uint16_t *router;     // [E + 1][H] bf16, the shared expert's gate row last
    const float *post_norm;
    float eps;
    float *logits;              // [M][E + 1]
    _Float16 *act_h;            // the experts' operands (act16 rows of the normalized x)
    int64_t act_stride;
    int H, E, E1, K;
    RouteState *rs;
    int32_t *ids_out;
    const StepParams *sp;
    int *ctr;                   // flags: [0, n_o) a projection workgroup done, [n_o, n_o + n_r) a router workgroup
    int *err;
    int n_o, n_r;
    int route_role;             // 1: the launch's last workgroup routes; 0: the experts' up launch routes the rows
                                // itself (and clears these flags)
};

template <int KW>
__device__ inline void mixout_o(const MixOutArgs &a, int wg, f4 *part, uint2 *tab) {
    trace(GV_K_O, 0);
    const int M = a.sp->M, H = a.H;
    const int64_t ntiles = tiles_rows(H);
    const int64_t t0 = static_cast<int64_t>(wg) * a.o_per;
    const int nt = static_cast<int>(std::min<int64_t>(a.o_per, ntiles - t0));
    const int o0 = threadIdx.x;
    const float g = a.o.global;
    // the thread's first output item (gemv_q4_kernel's order): its four rows of x loaded with the weights
    auto item = [&](int o, int64_t &row0, int &j) {
        const int i = o / 64, ll = o % 64;
        row0 = (t0 + i) * kTileR + 4 * (ll / 16);
        j = ll % 16;
    };
    float old[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto prefetch = [&] {
        int64_t row0;
        int j;
        item(min(o0, nt * 64 - 1), row0, j);
        const float *p = a.x + static_cast<int64_t>(min(j, M - 1)) * H;
#pragma unroll
        for (int r = 0; r < 4; ++r) old[r] = p[min(row0 + r, static_cast<int64_t>(H) - 1)];
    };
    if (nt > 0)
        mfma_tiles<KW, 1, kKeepParts, 0, 3, true>(
            a.o.codes, a.o.scales, H, static_cast<int>(a.o.cols / kSuperK), 0, nt, M,
            [&](int j) { return a.act_core + j * a.core_stride; }, [](int64_t, int, float) {}, part, tab, TileRun{t0},
            prefetch);
    const int W = blockDim.x / 64;
    for (int o = o0; o < nt * 64; o += blockDim.x) {   // the waves' partial sums in wave order, then x += sum x global
        const int i = o / 64, ll = o % 64;
        f4 sum = part[(i * W + 0) * 64 + ll];
        for (int w2 = 1; w2 < W; ++w2) sum += part[(i * W + w2) * 64 + ll];
        int64_t row0;
        int j;
        item(o, row0, j);
        if (j >= M || row0 >= H) continue;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float prev = o == o0 ? old[r] : a.x[j * static_cast<int64_t>(H) + row0 + r];
            v[r] = prev + sum[r] * g;
        }
        xst4f(a.x, static_cast<uint32_t>(j * H + row0), make_float4(v[0], v[1], v[2], v[3]));
    }
    trace(GV_K_O, 3);
    signal_done(a.ctr + wg);
}

// the router's part (router_kernel's arithmetic on 512 threads, rows of x read once the projection is done)
__device__ inline void mixout_router(const MixOutArgs &a, int wg, float *lds, double (*red)[4]) {
    trace(GV_K_ROUTER, 0);
    const int M = a.sp->M, H = a.H, ng = H / 8, steps = H / 8;
    const int tid = threadIdx.x, half = tid / 256, g = tid % 256, wave = tid / 64, lane = tid % 64;
    const int r0 = wg * 4;
    float *hT = lds;                          // [M][8][kRT]: row t, partial j: values j, j + 8, ... (step u = group)
    float *wT = hT + static_cast<size_t>(M) * 8 * kRT;   // [4][8][kRT]: the workgroup's router rows, the same order
    // before the wait: the router rows (4 x H bf16: two 16-byte loads a thread) and the norm weights
    const float *zero = reinterpret_cast<const float *>(g_zero_act16);
    uint4 wr[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = min(tid + k * 512, 4 * ng - 1), rr = i / ng, c8 = i % ng;
        wr[k] = *reinterpret_cast<const uint4 *>(a.router + static_cast<int64_t>(min(r0 + rr, a.E1 - 1)) * H + c8 * 8);
    }
    float nw[8];
    {
        const float *src = g < ng ? a.post_norm + g * 8 : zero;
        const float4 p = *reinterpret_cast<const float4 *>(src), q = *reinterpret_cast<const float4 *>(src + 4);
        const float t8[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) nw[i] = __fadd_rn(1.0f, t8[i]);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {   // the router rows into LDS as fp32, transposed: value c of row rr at chain c % 8, step c / 8
        const int i = tid + k * 512;
        if (i >= 4 * ng) break;
        const int rr = i / ng, c8 = i % ng;
        const uint32_t u[4] = {wr[k].x, wr[k].y, wr[k].z, wr[k].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            wT[(rr * 8 + 2 * e) * kRT + c8] = __uint_as_float(u[e] << 16);
            wT[(rr * 8 + 2 * e + 1) * kRT + c8] = __uint_as_float(u[e] & 0xFFFF0000u);
        }
    }
    trace(GV_K_ROUTER, 1);
    wait_flags(a.ctr, a.n_o, a.err);
    trace(GV_K_ROUTER, 2);
    // the rows of x (sc1: written by the projection in this launch): threads [0, 256) rows 0, 2, ..., [256, 512) rows
    // 1, 3, ...; group g of each (8 values)
    constexpr int kRowsPerHalf = kMaxRowsMixOut / 2;
    float xv[kRowsPerHalf][8];
#pragma unroll
    for (int q = 0; q < kRowsPerHalf; ++q) {
        const int t = min(half + 2 * q, M - 1);
        const float4 p = g < ng ? xld4f(a.x, static_cast<uint32_t>(t * H + g * 8)) : make_float4(0, 0, 0, 0);
        const float4 s = g < ng ? xld4f(a.x, static_cast<uint32_t>(t * H + g * 8 + 4)) : make_float4(0, 0, 0, 0);
        const float t8[8] = {p.x, p.y, p.z, p.w, s.x, s.y, s.z, s.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[q][i] = t8[i];
    }
    // per row: the double sum of squares (the thread's eight in order, the wave's, then the four waves' in order:
    // router_kernel's), 1 / RMS, x inv (1 + w) to LDS (transposed) and, for row wg, the experts' operands
#pragma unroll
    for (int q = 0; q < kRowsPerHalf; ++q) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += static_cast<double>(xv[q][i]) * static_cast<double>(xv[q][i]);
        ss = wave_sum(ss);
        if (lane == 0) red[half + 2 * q][wave % 4] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kRowsPerHalf; ++q) {
        const int t = half + 2 * q;
        if (t >= M) break;   // uniform over the half
        const double tot = ((red[t][0] + red[t][1]) + red[t][2]) + red[t][3];
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(H)), a.eps)));
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(__fmul_rn(xv[q][i], inv), nw[i]);
        const bool live = g < ng;
        if (live)
#pragma unroll
            for (int e = 0; e < 8; ++e) hT[(t * 8 + e) * kRT + g] = v[e];
        if (t == wg) act16_group(v, g, live, a.act_h + static_cast<int64_t>(wg) * a.act_stride);
    }
    __syncthreads();
    // the dots: wave w < 4 takes router row r0 + w, lane (t = lane / 8, j = lane % 8) partial j of row t in order
    const int ra = r0 + wave;
    if (wave < 4 && ra < a.E1) {
        const int t = lane / 8, j = lane % 8;
        const float4 *hp = reinterpret_cast<const float4 *>(hT + (min(t, M - 1) * 8 + j) * kRT);
        const float4 *wp = reinterpret_cast<const float4 *>(wT + (wave * 8 + j) * kRT);
        float acc = 0.0f;
        for (int u4 = 0; u4 < steps / 4; u4 += 4) {   // 16 steps' operands read ahead of their sums
            float4 hh[4], ww[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                hh[k] = hp[u4 + k];
                ww[k] = wp[u4 + k];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc = __fadd_rn(acc, __fmul_rn(ww[k].x, hh[k].x));
                acc = __fadd_rn(acc, __fmul_rn(ww[k].y, hh[k].y));
                acc = __fadd_rn(acc, __fmul_rn(ww[k].z, hh[k].z));
                acc = __fadd_rn(acc, __fmul_rn(ww[k].w, hh[k].w));
            }
        }
        // ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)) (bf16_row_dots)
        const float s1 = __fadd_rn(acc, __shfl_down(acc, 4, 64));
        const float s2 = __fadd_rn(s1, __shfl_down(s1, 1, 64));
        const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));
        if (j == 0 && t < M) xstf(a.logits, static_cast<uint32_t>(t * a.E1 + ra), s3);
    }
    trace(GV_K_ROUTER, 3);
    signal_done(a.ctr + a.n_o + wg);
}

// the route's part: the router's logits (sc1) into LDS, then route_kernel's route
__device__ inline void mixout_route(const MixOutArgs &a, float *lds) {
    const int M = a.sp->M, E1 = a.E1;
    wait_flags(a.ctr + a.n_o, a.n_r, a.err);
    float *lg = lds;   // [M][E1]
    for (int i = threadIdx.x; i < M * E1; i += blockDim.x) lg[i] = xldf(a.logits, static_cast<uint32_t>(i));
    int *ids = reinterpret_cast<int *>(lg + M * E1);
    int *cnt = ids + kMaxRows * 16, *start = cnt + 260, *slot_of = start + 260;
    unsigned *rows = reinterpret_cast<unsigned *>(slot_of + 260);
    __shared__ int wtot[2][16];
    clear_flags(a.ctr, a.n_o + a.n_r);   // every other workgroup has passed its waits: ready for the next step
    __syncthreads();
    route_all(lg, a.E, a.K, M, a.rs, a.ids_out, RouteLds{ids, cnt, start, slot_of, rows, wtot});
}

template <int KW>
__global__ __launch_bounds__(512) void mixout_kernel(const MixOutArgs a) {
    extern __shared__ uint4 mix_lds[];
    __shared__ uint2 tab[256];
    __shared__ double red[kMaxRowsMixOut][4];
    const int b = blockIdx.x;
    if (b < a.n_o) mixout_o<KW>(a, b, reinterpret_cast<f4 *>(mix_lds), tab);
    else if (b < a.n_o + a.n_r) mixout_router(a, b - a.n_o, reinterpret_cast<float *>(mix_lds), red);
    else if (a.route_role) mixout_route(a, reinterpret_cast<float *>(mix_lds));
}

// The experts' products on the matrix cores: UP takes gate_up [2F x H] against the post-norm rows of a slot's tokens,
// DOWN takes down [H x F] against the slot's picks' SwiGLU rows; each pick's rows go to out [pick][rows]. The grid is
// one round of resident workgroups; the slots' units (row tiles, or matched tile pairs with SW) are laid end to end
// and each workgroup takes an equal run of them, so a workgroup spans one or two slots (each part loading its
// slot's rows once) and the chip ends the launch together.
constexpr int kMoeFlush = 8;   // tiles whose partial sums an expert workgroup holds at once

// The SwiGLU of a matched gate / up tile pair's sums for F tile p (gs, us: the lane's rows 4 lg .. 4 lg + 3 of its
// column; x their globals g0, g1), m = silu(gate) x up (swiglu_quant_kernel's arithmetic), quantized per 16-value
// block (the pair's 16 rows: the column's four lanes) into the act16 operands of the column's row (live: the column
// is a pick). Every lane of the wave calls it (lane shuffles).
__device__ inline void swiglu_pair_out(f4 gs, f4 us, float g0, float g1, int p, bool live, _Float16 *row) {
    const int lg = (threadIdx.x % 64) / 16;
    float mv[4], amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = gs[r] * g0, uv = us[r] * g1;
        mv[r] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), uv);
        amax = fmaxf(amax, fabsf(mv[r]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float sc = __fdiv_rn(amax, 127.0f), qi = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    uint32_t hw[2], lw[2];   // this lane's 4 values (rows 4 lg .. 4 lg + 3 of the pair): hi, lo halves
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
    if ((lg & 1) == 0 && live) {
        auto inter = [](uint32_t mine, uint32_t other) {   // (m0, o0), (m1, o1) as two words
            return make_uint2((mine & 0xFFFFu) | (other << 16), (mine >> 16) | (other & 0xFFFF0000u));
        };
        const uint2 h01 = inter(hw[0], ph[0]), h23 = inter(hw[1], ph[1]);
        const uint2 l01 = inter(lw[0], pl[0]), l23 = inter(lw[1], pl[1]);
        const int gi = 2 * p + lg / 2;
        uint4 *dst = reinterpret_cast<uint4 *>(row + static_cast<int64_t>(gi) * 16);
        dst[0] = make_uint4(h01.x, h01.y, h23.x, h23.y);
        dst[1] = make_uint4(l01.x, l01.y, l23.x, l23.y);
    }
}

// SW (UP): the workgroup's tiles are matched gate / up pairs (gate tile p, up tile F / 16 + p: the tile loop takes
// them in turns, tiles_per_wg even), and each flush of two pairs writes their SwiGLU's operands for down
// (swiglu_pair_out) to sw_out [pick] instead of the products to out: no gate|up buffer, no SwiGLU launch.
template <int KW, int NTT, int WMAX, bool UP, bool SW = false>
__global__ __launch_bounds__(64 * WMAX) void moe_mfma_kernel(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales,
                                                        size_t code_stride, size_t scale_stride, int64_t rows, int K,
                                                        const float *__restrict__ globals, int half_rows,
                                                        const _Float16 *__restrict__ act, int64_t act_stride,
                                                        const float *__restrict__ gu, const Slots sl,
                                                        float *__restrict__ out, int E1, int max_picks,
                                                        _Float16 *__restrict__ sw_out, int64_t sw_stride) {
    static_assert(!SW || (UP && kMoeFlush % 2 == 0), "pairs: the up products, whole pairs a flush");
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    // (32-bit and uniform: slots x units stay far below 2^31 / the grid)
    const int ntiles = static_cast<int>(tiles_rows(rows)), npair = ntiles / 2, U = SW ? npair : ntiles;   // units a slot
    const int total = __builtin_amdgcn_readfirstlane(*sl.n_slots) * U, G = static_cast<int>(gridDim.x);
    const int x0 = static_cast<int>(blockIdx.x) * total / G, x1 = (static_cast<int>(blockIdx.x) + 1) * total / G;
    for (int x = x0; x < x1;) {   // (the same sequence in every thread)
        const int u = x / U, p0 = x - u * U, p1 = min(U, p0 + (x1 - x));
        x += p1 - p0;
        const int e = sl.expert[u], start = sl.start[u], cnt = sl.count[u];
        if (e < 0 || e >= E1 || cnt < 1 || cnt > kMaxRows || start < 0 || start + cnt > max_picks) continue;   // no slot
        const float g0 = globals[e * 3], g1 = globals[e * 3 + 1], g2 = globals[e * 3 + 2];
        if constexpr (SW) {   // pairs [p0, p1): gate tile p, up tile npair + p
            const int P0 = static_cast<int>(p0);
            mfma_tiles<KW, NTT, kSplitK, 0, 3, false, kMoeFlush>(
                codes + static_cast<size_t>(e) * code_stride, scales + static_cast<size_t>(e) * scale_stride, rows,
                K / kSuperK, 0, static_cast<int>(2 * (p1 - p0)), cnt,
                [&](int j) { return act + static_cast<int64_t>(sl.pick_token[start + j]) * act_stride; },
                [](int64_t, int, float) {}, part_lds, tab,
                [&](int i) -> int64_t { return (i & 1) ? npair + P0 + (i >> 1) : P0 + (i >> 1); }, NoHook{}, NoHook{},
                flush_with([&](int i0, int i1, const f4 *part, int W) {   // a pair and column tile a wave: sums in wave order
                    for (int o = threadIdx.x; o < (i1 - i0) / 2 * NTT * 64; o += blockDim.x) {
                        const int q = o / (NTT * 64), tt = (o / 64) % NTT, ll = o % 64;
                        f4 gs = part[((2 * q * W) * NTT + tt) * 64 + ll], us = part[(((2 * q + 1) * W) * NTT + tt) * 64 + ll];
                        for (int w2 = 1; w2 < W; ++w2) {
                            gs += part[(((2 * q) * W + w2) * NTT + tt) * 64 + ll];
                            us += part[(((2 * q + 1) * W + w2) * NTT + tt) * 64 + ll];
                        }
                        const int j = tt * 16 + ll % 16;
                        swiglu_pair_out(gs, us, g0, g1, P0 + (i0 >> 1) + q, j < cnt, sw_out + (start + j) * sw_stride);
                    }
                }));
        } else if constexpr (!UP) {   // down, tiles [p0, p1): a lane's four sums are four consecutive rows of its
                                      // pick's output, one 16-byte store (rows a multiple of 16)
            mfma_tiles<KW, NTT, kSplitK, 0, 3, false, kMoeFlush>(
                codes + static_cast<size_t>(e) * code_stride, scales + static_cast<size_t>(e) * scale_stride, rows,
                K / kSuperK, 0, p1 - p0, cnt, [&](int j) { return act + static_cast<int64_t>(start + j) * act_stride; },
                [](int64_t, int, float) {}, part_lds, tab, TileRun{p0}, NoHook{}, NoHook{},
                flush_with([&](int i0, int i1, const f4 *part, int W) {   // a tile and column tile a lane: wave order
                    for (int o = threadIdx.x; o < (i1 - i0) * NTT * 64; o += blockDim.x) {
                        const int i = o / (NTT * 64), tt = (o / 64) % NTT, ll = o % 64;
                        f4 sum = part[((i * W) * NTT + tt) * 64 + ll];
                        for (int w2 = 1; w2 < W; ++w2) sum += part[((i * W + w2) * NTT + tt) * 64 + ll];
                        const int j = tt * 16 + ll % 16;
                        const int64_t row = static_cast<int64_t>(p0 + i0 + i) * kTileR + 4 * (ll / 16);
                        if (j < cnt) *reinterpret_cast<f4 *>(out + static_cast<int64_t>(start + j) * rows + row) = sum * g2;
                    }
                }));
        } else {   // up, tiles [p0, p1)
            mfma_tiles<KW, NTT, kSplitK, 0, 3, false, kMoeFlush>(
                codes + static_cast<size_t>(e) * code_stride, scales + static_cast<size_t>(e) * scale_stride, rows,
                K / kSuperK, 0, static_cast<int>(p1 - p0), cnt,
                [&](int j) {   // UP: the row's act16 operands; DOWN: the pick's SwiGLU operands
                    const int64_t src = UP ? sl.pick_token[start + j] : start + j;
                    return act + src * act_stride;
                },
                [&](int64_t row, int j, float v) {
                    const float gl = UP ? (row < half_rows ? g0 : g1) : g2;
                    out[static_cast<int64_t>(start + j) * rows + row] = v * gl;
                },
                part_lds, tab, TileRun{p0});
        }
    }
}

// ---------------------------------------------------------------- the decode MoE
// The experts' products of the verify step's slots (runs of at most kSlotRows picks of one expert), in two launches.
// Up: a workgroup per (slot, kMoePairs matched gate/up row tile pairs); its waves split K = H, and it computes gate
// tile p and up tile p together, so the 16 values m = silu(gate) x up of a tile pair and their 16-value quantization
// block are its own: it writes the picks' down operands (act16) directly (no gate|up buffer, no SwiGLU launch). Down:
// a workgroup per (slot, group of row tiles), each wave kMoeDnTiles tiles over the whole K = F. Every tile loop is
// unrolled (mfma_tiles with a fixed tile count).
constexpr int kMoePairs = 3;       // tile pairs an up workgroup takes
constexpr int kMoeDnTiles = 2;     // down tiles a wave takes

struct MoeArgsDec {
    const uint8_t *gu_codes, *gu_scales, *dn_codes, *dn_scales;
    size_t gu_cstride, gu_sstride, dn_cstride, dn_sstride;
    int H, F;
    const float *globals;                 // [E + 1][3]
    const _Float16 *act;                  // the rows' operands (act16, act_stride halves apart)
    int64_t act_stride;
    _Float16 *act_m;                      // the picks' down operands (act16, F values a pick)
    float *y;                             // [pick][H]
    Slots sl;
    int groups, E1, max_picks;
    // the route made by the up launch itself (moe_up_kernel<KWU, true>): the rows' router logits [M][E1], the route
    // state its workgroup 0 writes for the launches after it, the routed ids out, and the previous launch's flags
    // (the fused output projection / router's) that workgroup 0 clears for the next step
    const float *logits;
    int E, K;
    RouteState *rs;
    int32_t *ids_out;
    const StepParams *sp;
    int *flags;
    int n_flags;
};

// the slot of this workgroup (blockIdx / groups) and its expert, first pick and pick count, and the lane's pick's
// row (pick lane % 8 of the slot; a lane past the count: the slot's first): all loaded at once (the slot's entries
// are read before knowing it is live; every index is inside the route state); false: no slot
__device__ inline bool moe_slot(const MoeArgsDec &a, int u, int &e, int &start, int &cnt, int &tok) {
    const int ns = *a.sl.n_slots;
    e = a.sl.expert[u], start = a.sl.start[u], cnt = a.sl.count[u];
    tok = a.sl.token[u * kSlotRows + (threadIdx.x % 64) % 8];
    return u < ns && e >= 0 && e < a.E1 && cnt >= 1 && cnt <= kSlotRows && start >= 0 && start + cnt <= a.max_picks &&
           tok >= 0 && tok < kMaxRows;
}

// ROUTE: the launch routes the rows itself (at most kMaxRowsMixOut of them): every workgroup runs the route on the
// router's logits into its LDS (route_core: the same ids, counts and scans whichever workgroup runs it) and takes its
// slot from there, so that no route launch or hand-off sits between the router and the experts; workgroup 0 also
// writes the route state (the down products, the combine and the ids read it after this launch) and clears the
// router launch's flags. Otherwise the slot comes from the route state the route launch wrote.
template <int KWU, bool ROUTE>
__global__ __launch_bounds__(512) void moe_up_kernel(const MoeArgsDec a) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    trace(GV_K_MOE_UP, 0);
    const int u = static_cast<int>(blockIdx.x) / a.groups, grp = static_cast<int>(blockIdx.x) % a.groups;
    int e, start, cnt, tok;
    if constexpr (ROUTE) {
        __shared__ int r_ids[kMaxRowsMixOut * 16], r_cnt[260], r_start[260], r_slot[260], r_sel[4];
        __shared__ unsigned r_rows[260];
        __shared__ int r_wtot[2][16];
        const RouteLds r{r_ids, r_cnt, r_start, r_slot, r_rows, r_wtot};
        const bool writer = blockIdx.x == 0;
        const int M = a.sp->M;
        route_small(a.logits, a.E, a.K, M, writer ? a.rs->weight : nullptr, writer ? a.rs->gate : nullptr, r, u,
                    r_sel);
        if (writer) {
            route_tables(a.E, a.K, M, a.rs, a.ids_out, r);
            clear_flags(a.flags, a.n_flags);   // (every workgroup of the router's launch is done: it came before)
        }
        e = r_sel[0];
        if (e < 0) return;   // (uniform: LDS)
        start = r_sel[1], cnt = r_sel[2];
        const int j = (threadIdx.x % 64) % 8, nth = j < cnt ? j : 0;   // the lane's pick (past the count: the first)
        if (e == a.E) {
            tok = nth;   // (the shared expert: every row, in order)
        } else {
            uint32_t mk = static_cast<uint32_t>(r_sel[3]);
            for (int i = 0; i < nth; ++i) mk &= mk - 1u;   // the nth-lowest set bit: the rows in order
            tok = __builtin_ctz(mk);
        }
    } else {
        if (!__builtin_amdgcn_readfirstlane(moe_slot(a, u, e, start, cnt, tok))) return;
    }
    trace(GV_K_MOE_UP, 4);
    const int F = a.F, W = blockDim.x / 64, lane = threadIdx.x % 64;
    const int64_t act_m_stride = act_halves(F);
    const int npair = F / kTileR, p0 = grp * kMoePairs, np = min(kMoePairs, npair - p0);
    if (np <= 0) return;
    mfma_tiles<KWU, 1, kKeepParts, 2 * kMoePairs, 3, true>(
        a.gu_codes + static_cast<size_t>(e) * a.gu_cstride, a.gu_scales + static_cast<size_t>(e) * a.gu_sstride,
        2 * F, a.H / kSuperK, 0, 2 * np, cnt,
        [&](int) { return a.act + static_cast<int64_t>(tok) * a.act_stride; },   // (packed: j = lane % 8)
        [](int64_t, int, float) {}, part_lds, tab,
        [&](int i) -> int64_t { return (i & 1) ? npair + p0 + (i >> 1) : p0 + (i >> 1); }, NoHook{},
        [] { trace(GV_K_MOE_UP, 5); });
    trace(GV_K_MOE_UP, 1);
    const float g0 = a.globals[e * 3], g1 = a.globals[e * 3 + 1];
    // per pair (a wave each): the waves' sums in wave order, x global (the products' put), then m = silu(gate) x up
    // (swiglu_quant_kernel's arithmetic) and the 16-value block's operands
    for (int o = threadIdx.x; o < np * 64; o += blockDim.x) {
        const int q = o / 64, j = lane % 16, lg = lane / 16;
        f4 gs = part_lds[(2 * q * W) * 64 + lane], us = part_lds[((2 * q + 1) * W) * 64 + lane];
        for (int w2 = 1; w2 < W; ++w2) {
            gs += part_lds[(2 * q * W + w2) * 64 + lane];
            us += part_lds[((2 * q + 1) * W + w2) * 64 + lane];
        }
        swiglu_pair_out(gs, us, g0, g1, p0 + q, j < cnt, a.act_m + (start + j) * act_m_stride);
    }
    trace(GV_K_MOE_UP, 3);
}

template <int KWD>
__global__ __launch_bounds__(256) void moe_down_kernel(const MoeArgsDec a) {
    __shared__ uint2 tab[256];
    trace(GV_K_MOE_DOWN, 0);
    const int u = static_cast<int>(blockIdx.x) / a.groups, grp = static_cast<int>(blockIdx.x) % a.groups;
    int e, start, cnt, tok;
    const int dst = a.sl.dst[u * kSlotRows + (threadIdx.x % 64) % 8];   // the lane's pick's output row
    if (!__builtin_amdgcn_readfirstlane(moe_slot(a, u, e, start, cnt, tok))) return;
    trace(GV_K_MOE_DOWN, 4);
    const int H = a.H, F = a.F, W = blockDim.x / 64, w = threadIdx.x / 64;
    const int64_t act_m_stride = act_halves(F);
    const int wt0 = (grp * W + w) * kMoeDnTiles, nt = max(0, min(kMoeDnTiles, H / kTileR - wt0));
    const float g2 = a.globals[e * 3 + 2];
    mfma_tiles<KWD, 1, kWaveTiles, kMoeDnTiles, kMoeDnTiles, true>(
        a.dn_codes + static_cast<size_t>(e) * a.dn_cstride, a.dn_scales + static_cast<size_t>(e) * a.dn_sstride, H,
        F / kSuperK, 0, nt, cnt,
        [&](int j) { return a.act_m + (start + j) * act_m_stride; },
        [&](int64_t row, int, float v) { a.y[static_cast<int64_t>(dst) * H + row] = v * g2; },   // (j = lane % 16)
        nullptr, tab,
        TileRun{wt0}, NoHook{}, [] { trace(GV_K_MOE_DOWN, 5); });
    trace(GV_K_MOE_DOWN, 3);
}

// per pick: silu(gate) * up (kernels.hpp:141), quantized for down
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float *__restrict__ gu, int F,
                                                           const int *__restrict__ n_picks,
                                                           _Float16 *__restrict__ act_m) {
    extern __shared__ uint4 lds_u4[];
    float *m = reinterpret_cast<float *>(lds_u4);
    const int p = blockIdx.x;
    if (p >= *n_picks) return;
    const float *row = gu + static_cast<int64_t>(p) * 2 * F;
    for (int i = threadIdx.x; i < F; i += blockDim.x) {
        const float x = row[i];
        m[i] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), row[F + i]);
    }
    __syncthreads();
    norm_quant_row(m, F, nullptr, 0.0f, act_m + static_cast<int64_t>(p) * act_halves(F), nullptr, nullptr);
}

// x += sigmoid(gate) x shared + sum_k w_k y_k in rank order (model.cpp:4554-4585, :5363-5365); a workgroup per
// (row, 256 columns)
// x += sigmoid(gate) x shared + sum_k w_k y_k in rank order (model.cpp:4554-4585, :5363-5365), then the next RMSNorm
// and its operands; a workgroup per row
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y, int H, int K, const MixView mix,
                                                      int M, float *__restrict__ x, const float *__restrict__ norm_w,
                                                      float eps, _Float16 *__restrict__ act, int64_t act_stride,
                                                      float *__restrict__ hout, int residual) {
    __shared__ double red[16];
    const int t = blockIdx.x;
    if (t >= M) return;
    const int ng = H / 8;
    const float *zero = reinterpret_cast<const float *>(g_zero_act16);
    const float gs = mix.gate[t];
    auto row_of = [&](int k) { return mix.pick_of ? mix.pick_of[t * (K + 1) + k] : t * (K + 1) + k; };
    const float *ysh = y + static_cast<int64_t>(row_of(K)) * H;
    // Every load of a group of eight values issued before the first use (indices clamped, no branch around a
    // load): the next norm's weights, the shared expert's row, the first eight picks' rows (picks past K read pick
    // K - 1 and are not added), the residual row.
    float w1[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * blockDim.x;
        const float *src = norm_w && g < ng ? norm_w + g * 8 : zero;
        const float4 a = *reinterpret_cast<const float4 *>(src), b = *reinterpret_cast<const float4 *>(src + 4);
        const float tw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) w1[q][i] = __fadd_rn(1.0f, tw[i]);
    }
    float v[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[q][i] = 0.0f;
        if (q * static_cast<int>(blockDim.x) >= ng) continue;   // uniform
        const int g = threadIdx.x + q * blockDim.x, gc = min(g, ng - 1);
        const bool live = g < ng;
        float4 ya[9], yb[9];
        ya[8] = *reinterpret_cast<const float4 *>(ysh + gc * 8);
        yb[8] = *reinterpret_cast<const float4 *>(ysh + gc * 8 + 4);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float *yk = y + static_cast<int64_t>(row_of(min(u, K - 1))) * H + gc * 8;
            ya[u] = *reinterpret_cast<const float4 *>(yk);
            yb[u] = *reinterpret_cast<const float4 *>(yk + 4);
        }
        float *xr = x + static_cast<int64_t>(t) * H + gc * 8;
        const float *xs = residual ? xr : zero + gc * 8;   // (no residual: the block's output alone, x + 0)
        const float4 xa = *reinterpret_cast<const float4 *>(xs), xb = *reinterpret_cast<const float4 *>(xs + 4);
        float wkv[8];   // the picks' weights, with the rows (not a round trip after them)
#pragma unroll
        for (int u = 0; u < 8; ++u) wkv[u] = mix.weight[t * K + min(u, K - 1)];
        __builtin_amdgcn_sched_barrier(0);
        float o[8];
        {
            const float yv[8] = {ya[8].x, ya[8].y, ya[8].z, ya[8].w, yb[8].x, yb[8].y, yb[8].z, yb[8].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = __fmul_rn(gs, yv[i]);
        }
        // rank order, skipping zero weights
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float wk = u < K ? wkv[u] : 0.0f;
            if (wk == 0.0f) continue;   // uniform
            const float yv[8] = {ya[u].x, ya[u].y, ya[u].z, ya[u].w, yb[u].x, yb[u].y, yb[u].z, yb[u].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = __fadd_rn(o[i], __fmul_rn(wk, yv[i]));
        }
        for (int k = 8; k < K; ++k) {   // more than eight picks a row: one at a time
            const float wk = mix.weight[t * K + k];
            if (wk == 0.0f) continue;
            const float *yk = y + static_cast<int64_t>(row_of(k)) * H + gc * 8;
            const float4 a = *reinterpret_cast<const float4 *>(yk), b = *reinterpret_cast<const float4 *>(yk + 4);
            const float yv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = __fadd_rn(o[i], __fmul_rn(wk, yv[i]));
        }
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[q][i] = live ? __fadd_rn(xv[i], o[i]) : 0.0f;
        if (live) {
            *reinterpret_cast<float4 *>(xr) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
            *reinterpret_cast<float4 *>(xr + 4) = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
        }
    }
    if (act)
        norm_quant_regs_w(v, H, norm_w != nullptr, w1, eps, act + static_cast<int64_t>(t) * act_stride,
                          hout ? hout + static_cast<int64_t>(t) * H : nullptr, red);
}

// (hout: the normalized rows in fp32 too, [M][H], or null)
// (residual false: x is written, not read: the block's output without a residual)
inline int combine_launch(const float *y, int H, int K, const MixView &mix, int M, float *x, const float *norm_w,
                          float eps, _Float16 *act, int64_t act_stride, hipStream_t st, float *hout = nullptr,
                          bool residual = true) {
    hipLaunchKernelGGL(combine_kernel, dim3(M), dim3(256), 0, st, y, H, K, mix, M, x, norm_w, eps, act, act_stride,
                       hout, residual ? 1 : 0);
    return 0;
}

// the fused projection + router + route (mixout_kernel) where the shapes fit it: at most 8 rows, hidden <= 2048, the
// projection's K split over exactly the launch's 8 waves
// (o_cols: the output projection's input width, n_heads x head_dim or a Gated DeltaNet layer's nv x dv)
inline bool mixout_fits(const Model &m, int M, int64_t o_cols, int &kw) {
    const auto &c = m.c;
    if (!m.fused || m.moe_only || M > kMaxRowsMixOut || c.hidden > 2048 || c.hidden % kSuperK || m.E1 > 257) return false;
    int waves = 0;
    if (!mfma_split(o_cols, 1, waves, kw) || waves != 8) return false;
    return kw == 16 || kw == 8 || kw == 4;
}

// the flags of the fused output projection / router launch: its projection workgroups' and its router workgroups'
inline int mixout_flags(const Model &m) {
    const int64_t ntiles = tiles_rows(m.c.hidden);
    const int64_t per = tiles_per_wg(ntiles, 8, 1);
    return static_cast<int>((ntiles + per - 1) / per) + (m.E1 + 3) / 4;
}

inline size_t mixout_lds(int M, int E1, int o_per) {
    const size_t router = static_cast<size_t>(M + 4) * 8 * kRT * 4;
    const size_t route = (static_cast<size_t>(M) * E1 + kMaxRows * 16 + 4 * 260) * 4;
    const size_t o = static_cast<size_t>(o_per) * 8 * 1024;
    return std::max({router, route, o});
}

// verify_keep of a tree: the kept path's keys and values moved to the kept slots in every layer; a thread per
// (layer, KV head, dim)
// (T: _Float16, or int8_t for the int8 cache, whose scales follow each layer's values: dim 0's thread moves them)
template <typename T>
__global__ void kv_compact_kernel(uint8_t *kv_all, size_t layer_bytes, int n_layers, int nkv, int hd, int64_t slots,
                                  int pos, int kept, const int *__restrict__ path) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(n_layers) * nkv * hd) return;
    const int l = static_cast<int>(i / (static_cast<int64_t>(nkv) * hd)), kh = static_cast<int>((i / hd) % nkv);
    const int d = static_cast<int>(i % hd);
    T *kv = reinterpret_cast<T *>(kv_all + static_cast<size_t>(l) * layer_bytes);
    float *sc = reinterpret_cast<float *>(kv + 2 * static_cast<int64_t>(nkv) * slots * hd);
    for (int j = 1; j < kept; ++j) {   // ascending: path[j] >= j, so no source is overwritten before it is read
        if (path[j] == j) continue;
        kv[k_index(slots, hd, kh, pos + j, d)] = kv[k_index(slots, hd, kh, pos + path[j], d)];
        kv[v_index(slots, hd, nkv, kh, pos + j, d)] = kv[v_index(slots, hd, nkv, kh, pos + path[j], d)];
        if (sizeof(T) == 1 && d == 0)
            for (int w = 0; w < 2; ++w)
                sc[kv_scale_index(slots, nkv, w, kh, pos + j)] = sc[kv_scale_index(slots, nkv, w, kh, pos + path[j])];
    }
}

// positions [0, n) of the reference's layout ([K, V][position][nkv * hd], fp32 here) into the device layout
__global__ void kv_from_rows_kernel(const float *__restrict__ src, int n, int nkv, int hd, int64_t slots,
                                    _Float16 *__restrict__ kv) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t kv_row = static_cast<int64_t>(nkv) * hd;
    if (i >= 2 * n * kv_row) return;
    const int which = static_cast<int>(i / (n * kv_row));
    const int p = static_cast<int>((i / kv_row) % n);
    const int kh = static_cast<int>((i % kv_row) / hd), d = static_cast<int>(i % hd);
    const _Float16 v = static_cast<_Float16>(src[i]);
    if (which == 0) kv[k_index(slots, hd, kh, p, d)] = v;
    else kv[v_index(slots, hd, nkv, kh, p, d)] = v;
}

// the int8 cache from fp32 rows ([K, V][position][nkv * hd], positions [0, n)): quant_kv_row of each (K or V,
// position, KV head) row, a workgroup (256 threads, hd <= 256) a row
__global__ __launch_bounds__(256) void kv8_from_rows_kernel(const float *__restrict__ src, int n, int nkv, int hd,
                                                            int64_t slots, int8_t *__restrict__ kv8,
                                                            float *__restrict__ kvs) {
    __shared__ float red4[4];
    const int row = blockIdx.x, which = row / (n * nkv), p = (row / nkv) % n, kh = row % nkv, d = threadIdx.x;
    const bool live = d < hd;
    const float x = live ? src[(static_cast<int64_t>(which) * n + p) * nkv * hd + static_cast<int64_t>(kh) * hd + d] : 0.0f;
    int8_t *q = kv8 + (which == 0 ? k_index(slots, hd, kh, p, d) : v_index(slots, hd, nkv, kh, p, d));
    const float sc = kv_quant_row(x, red4, q, live);
    if (d == 0) kvs[kv_scale_index(slots, nkv, which, kh, p)] = sc;
}

// the int8 cache from the reference's int8 rows: int8 [K, V][position][nkv * hd] and float [K, V][position][nkv]
__global__ void kv8_copy_kernel(const int8_t *__restrict__ src, const float *__restrict__ ssrc, int n, int nkv, int hd,
                                int64_t slots, int8_t *__restrict__ kv8, float *__restrict__ kvs) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t kv_row = static_cast<int64_t>(nkv) * hd;
    if (i >= 2 * n * kv_row) return;
    const int which = static_cast<int>(i / (n * kv_row));
    const int p = static_cast<int>((i / kv_row) % n);
    const int kh = static_cast<int>((i % kv_row) / hd), d = static_cast<int>(i % hd);
    kv8[which == 0 ? k_index(slots, hd, kh, p, d) : v_index(slots, hd, nkv, kh, p, d)] = src[i];
    if (d == 0) kvs[kv_scale_index(slots, nkv, which, kh, p)] = ssrc[(static_cast<int64_t>(which) * n + p) * nkv + kh];
}

__global__ void f32_to_bf16_kernel(const float *__restrict__ x, int64_t n, uint16_t *__restrict__ y) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t u = __float_as_uint(x[i]);
    u = u + 0x7FFFu + ((u >> 16) & 1u);
    y[i] = static_cast<uint16_t>(u >> 16);
}

__global__ void f32_to_f16_kernel(const float *__restrict__ x, int64_t n, uint16_t *__restrict__ y) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x[i]));
}

// ---------------------------------------------------------------- launches
namespace {

// the slots a step of M rows can have: its distinct experts (at most M K) and the shared one
inline int moe_slots_bound(int E, int K, int M) { return std::min(E, M * K) + 1 + M * (K + 1) / kSlotRows; }
inline int moe_slots(const Model &m, int M) { return std::min(m.max_slots, moe_slots_bound(m.c.n_experts, m.c.top_k, M)); }

// One launch of the experts' products over a slot list
struct MoeArgs {
    const uint8_t *codes, *scales;
    size_t code_stride, scale_stride;
    int64_t rows, cols;
    const float *globals;
    int F;
    const _Float16 *act;   // UP: the rows' operands, by pick_token
    const float *gu;       // DOWN: the picks' gate|up products (their SwiGLU quantized on the fly)
    Slots sl;
    float *out;            // [pick][rows]
    int slots;             // a bound on the slot count (the grid)
    int E1, max_picks;
    _Float16 *sw_out;      // UP with the SwiGLU in the launch: the picks' down operands (act16 rows of F), else null
};

template <int KW, int NTT, int WMAX, bool UP, bool SW>
int launch_moe_raw(const MoeArgs &a, int waves, hipStream_t st) {
    // one round of resident workgroups (2 waves a SIMD at these kernels' register use), the slots' units split
    // evenly among them on the device (the slot count is the route's)
    const int G = 256 * std::max(1, 8 / waves);
    const size_t lds = static_cast<size_t>(kMoeFlush) * waves * NTT * 1024;   // the waves' partial sums
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&moe_mfma_kernel<KW, NTT, WMAX, UP, SW>), std::max<size_t>(lds, 76 * 1024),
                  granted) != 0)
        return -1;
    hipLaunchKernelGGL((moe_mfma_kernel<KW, NTT, WMAX, UP, SW>), dim3(G), dim3(64 * waves), lds, st, a.codes, a.scales,
                       a.code_stride, a.scale_stride, a.rows, static_cast<int>(a.cols), a.globals, a.F, a.act,
                       act_halves(a.cols), a.gu, a.sl, a.out, a.E1, a.max_picks, a.sw_out, act_halves(a.F));
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

template <bool UP, bool SW = false>
int moe_launch(const MoeArgs &a, int ntt, int kw, int waves, hipStream_t st) {
    if (ntt == 1) {
        if (kw == 16) return launch_moe_raw<16, 1, 8, UP, SW>(a, waves, st);
        if (kw == 8) return launch_moe_raw<8, 1, 8, UP, SW>(a, waves, st);
        return launch_moe_raw<4, 1, 8, UP, SW>(a, waves, st);
    }
    if (kw == 8) return launch_moe_raw<8, 2, 8, UP, SW>(a, waves, st);
    return launch_moe_raw<4, 2, 8, UP, SW>(a, waves, st);
}

// the experts' products of layer L: gate|up (up) or down, over slots of at most `rows_max` rows each
// (sw_out: up with the SwiGLU in the launch, its operands for down to sw_out; null: the products to out)
int moe_run(const Model &m, const LayerW &L, bool up, int rows_max, const _Float16 *act, const float *gu,
            const Slots &sl, float *out, int slots, int max_picks, hipStream_t st, _Float16 *sw_out = nullptr) {
    const int64_t H = m.c.hidden, F = m.c.moe_ff;
    const int ntt = rows_max <= 16 ? 1 : 2;
    int waves, kw;
    GV_REQUIRE(mfma_split(up ? H : F, ntt, waves, kw), "moe: K too wide for one launch");
    MoeArgs a{up ? L.gu_codes : L.dn_codes,
              up ? L.gu_scales : L.dn_scales,
              up ? m.gu_code_stride : m.dn_code_stride,
              up ? m.gu_scale_stride : m.dn_scale_stride,
              up ? 2 * F : H,
              up ? H : F,
              L.expert_globals,
              static_cast<int>(F),
              act,
              gu,
              sl,
              out,
              slots,
              m.E1,
              max_picks,
              sw_out};
    if (up && sw_out) return moe_launch<true, true>(a, ntt, kw, waves, st);
    return up ? moe_launch<true>(a, ntt, kw, waves, st) : moe_launch<false>(a, ntt, kw, waves, st);
}

int moe_products(const Model &m, const LayerW &L, int M, bool up, hipStream_t st) {
    return moe_run(m, L, up, std::min(M, kSlotRows), up ? m.act_h : m.act_m, m.gu_out,
                   route_slots(m.route + (&L - &m.layers[0])), up ? m.gu_out : m.y, moe_slots(m, M), m.max_picks, st);
}

// The decode MoE kernels' shape: the up workgroup's waves split K = H (mfma_split's choice for 16-row tiles, at most
// 4 waves) and each down wave takes K = F whole; false when the shapes fall outside the compiled variants (the
// general products and the SwiGLU launch, moe_products, then run instead).
bool moe_dec_shape(const gv_model_config &c, int &kwu, int &kwd, int &waves) {
    const int64_t H = c.hidden, F = c.moe_ff;
    if (H % kSuperK || F % kSuperK || H % kTileR) return false;
    if (!mfma_split(H, 1, waves, kwu) || waves > 4) return false;
    kwd = static_cast<int>(F / 32);
    return (kwu == 16 && kwd == 16) || (kwu == 4 && kwd == 4);
}

// the decode up launch's threads (moe_dec's choice below)
int moe_up_threads(const gv_model_config &c) {
    int kwu, kwd, waves;
    if (!moe_dec_shape(c, kwu, kwd, waves)) return 0;
    return kwu == 16 && waves <= 4 ? 128 * waves : 64 * waves;
}

// whether the experts' up launch after the fused output projection / router launch routes the rows itself (the decode
// variant; route_small's bounds: at most 8 picks a row, 256 experts; not a replay of one launch alone); otherwise the
// fused launch keeps its route workgroup
inline bool up_routes(const Model &m, bool mixout) {
    return (mixout || m.block_up_routes) && m.route_in_up && m.moe_dec && !m.replaying && m.c.top_k <= 8 &&
           m.c.n_experts <= 256 && moe_up_threads(m.c) >= 64;
}

int moe_dec(const Model &m, const LayerW &L, int M, bool up, bool route, hipStream_t st) {
    int kwu, kwd, waves;
    GV_REQUIRE(moe_dec_shape(m.c, kwu, kwd, waves), "moe: no decode variant for this shape");
    GV_REQUIRE(!route || (up && M <= kMaxRowsMixOut), "moe: the up launch routes at most kMaxRowsMixOut rows");
    MoeArgsDec a{};
    a.gu_codes = L.gu_codes, a.gu_scales = L.gu_scales, a.dn_codes = L.dn_codes, a.dn_scales = L.dn_scales;
    a.gu_cstride = m.gu_code_stride, a.gu_sstride = m.gu_scale_stride;
    a.dn_cstride = m.dn_code_stride, a.dn_sstride = m.dn_scale_stride;
    a.H = m.c.hidden, a.F = m.c.moe_ff;
    a.globals = L.expert_globals;
    a.act = m.act_h, a.act_stride = act_halves(m.c.hidden);
    a.act_m = m.act_m;
    a.y = m.y;
    const int64_t l = &L - &m.layers[0];
    a.sl = route_slots(m.route + l);
    a.E1 = m.E1, a.max_picks = m.max_picks;
    a.logits = m.block_logits ? m.block_logits : m.rlogits, a.E = m.c.n_experts, a.K = m.c.top_k;
    a.rs = m.route + l;
    a.ids_out = m.route_ids + l * m.c.max_rows * m.c.top_k;
    a.sp = m.sp;
    a.flags = m.ctr + l * kFlagsPerLayer;
    a.n_flags = mixout_flags(m);
    const int slots = moe_slots(m, M);
    if (up) {
        a.groups = (a.F / kTileR + kMoePairs - 1) / kMoePairs;
        const dim3 grid(static_cast<unsigned>(slots * a.groups));
        if (kwu == 16 && waves <= 4) {   // eight waves, each half the K range
            const size_t lds = static_cast<size_t>(2 * kMoePairs) * (2 * waves) * 1024;
            if (route) hipLaunchKernelGGL((moe_up_kernel<8, true>), grid, dim3(128 * waves), lds, st, a);
            else hipLaunchKernelGGL((moe_up_kernel<8, false>), grid, dim3(128 * waves), lds, st, a);
        } else {
            const size_t lds = static_cast<size_t>(2 * kMoePairs) * waves * 1024;
            if (kwu == 16) {
                if (route) hipLaunchKernelGGL((moe_up_kernel<16, true>), grid, dim3(64 * waves), lds, st, a);
                else hipLaunchKernelGGL((moe_up_kernel<16, false>), grid, dim3(64 * waves), lds, st, a);
            } else {
                if (route) hipLaunchKernelGGL((moe_up_kernel<4, true>), grid, dim3(64 * waves), lds, st, a);
                else hipLaunchKernelGGL((moe_up_kernel<4, false>), grid, dim3(64 * waves), lds, st, a);
            }
        }
    } else {
        // a wave a workgroup (its tiles need no other wave): the finest grain, so that the CUs' shares even out
        a.groups = (a.H / kTileR + kMoeDnTiles - 1) / kMoeDnTiles;
        const dim3 grid(static_cast<unsigned>(slots * a.groups));
        if (kwd == 16) hipLaunchKernelGGL(moe_down_kernel<16>, grid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL(moe_down_kernel<4>, grid, dim3(64), 0, st, a);
    }
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// ---------------------------------------------------------------- prefill MoE (C5): many rows
// the shared expert's gate logit of each row (gate_row_logit); a wave a row
__global__ __launch_bounds__(256) void gate_rows_kernel(const uint16_t *__restrict__ wrow, int H,
                                                        const float *__restrict__ h, int M, float *__restrict__ logits,
                                                        int E1) {
    extern __shared__ float gr_lds[];
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const float s3 = gate_row_logit(wrow, H, h, M, t, gr_lds);
    if (t < M && lane == 0) logits[static_cast<int64_t>(t) * E1 + E1 - 1] = s3;
}

// route_topk of every row (route_row), a wave a row
__global__ __launch_bounds__(256) void route_rows_kernel(const float *__restrict__ logits, int E, int K, int M,
                                                         int *__restrict__ ids, float *__restrict__ w,
                                                         float *__restrict__ gate) {
    const int wave = threadIdx.x >> 6, t = blockIdx.x * 4 + wave;
    if (t >= M) return;
    route_row(logits + static_cast<int64_t>(t) * (E + 1), E, K, ids + static_cast<int64_t>(t) * K,
              w + static_cast<int64_t>(t) * K, gate + t);
}

// The picks per expert (the shared one, E, takes every row), their starts, and the slots: each expert's picks in
// runs of at most 32 (the products' row tiles), experts ascending. One workgroup of 1024 threads (E + 1 <= 257).
__global__ __launch_bounds__(1024) void group_kernel(const int *__restrict__ ids, int M, int K, int E,
                                                     int *__restrict__ start_out, int *__restrict__ n_slots,
                                                     int *__restrict__ slot_expert, int *__restrict__ slot_start,
                                                     int *__restrict__ slot_count, int *__restrict__ n_picks) {
    __shared__ int cnt[257], start[257], sbase[257];
    __shared__ int wt[2][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e <= E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int i = tid; i < M * K; i += blockDim.x) atomicAdd(&cnt[ids[i]], 1);
    if (tid == 0) cnt[E] = M;
    __syncthreads();
    const int c = tid <= E ? cnt[tid] : 0, ns = (c + 31) / 32;
    int ic = c, is = ns;
    for (int o = 1; o < 64; o <<= 1) {
        const int pc = __shfl_up(ic, o, 64), ps = __shfl_up(is, o, 64);
        if (lane >= o) ic += pc, is += ps;
    }
    if (lane == 63) wt[0][wave] = ic, wt[1][wave] = is;
    __syncthreads();
    if (tid <= E) {
        int bc = 0, bs = 0;
        for (int w2 = 0; w2 < wave; ++w2) bc += wt[0][w2], bs += wt[1][w2];
        start[tid] = bc + ic - c;
        sbase[tid] = bs + is - ns;
        start_out[tid] = bc + ic - c;
        if (tid == E) *n_slots = bs + is, *n_picks = bc + ic;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += blockDim.x)
        for (int j = 0; 32 * j < cnt[e]; ++j) {
            const int u = sbase[e] + j;
            slot_expert[u] = e;
            slot_start[u] = start[e] + 32 * j;
            slot_count[u] = min(32, cnt[e] - 32 * j);
        }
}

// The picks of expert blockIdx.x (fill_expert_picks)
__global__ __launch_bounds__(256) void fill_picks_kernel(const int *__restrict__ ids, int M, int K, int E,
                                                         const int *__restrict__ start, int *__restrict__ pick_token,
                                                         int *__restrict__ pick_of) {
    __shared__ int wt[kFillBatch][4];
    fill_expert_picks(ids, M, K, E, static_cast<int>(blockIdx.x), start[blockIdx.x], pick_token, pick_of, wt);
}

GemvOut qkv_out(const Model &m, const LayerW &L) {
    const auto &c = m.c;
    GemvOut o;
    o.y = m.qkv_out;
    o.ldy = L.qkv.rows;
    o.accumulate = 0;
    o.nseg = 3;
    o.seg_end[0] = static_cast<int64_t>(c.n_heads) * 2 * c.head_dim;
    o.seg_end[1] = o.seg_end[0] + static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
    o.seg_end[2] = INT64_MAX;
    o.seg_global[0] = L.g_q;
    o.seg_global[1] = L.g_k;
    o.seg_global[2] = L.g_v;
    return o;
}

// events around the launches of the timed kernel class
struct Tick {
    Model &m;
    int cls;
    hipStream_t st;
    bool on;
    Tick(Model &mm, int c, hipStream_t s) : m(mm), cls(c), st(s), on(mm.timed_class == c) { mark(); }
    ~Tick() { mark(); }
    void mark() {
        if (!on) return;
        if (m.events_used == m.events.size()) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) {
                on = false;
                return;
            }
            m.events.push_back(e);
        }
        (void)hipEventRecord(m.events[m.events_used++], st);
    }
};

template <int NCH, bool I8>
int launch_attn_t(Model &m, LayerW &L, hipStream_t st) {
    const auto &c = m.c;
    static int granted = 0;
    const size_t lds = attn_lds(NCH * 32);
    if (lds_grant(reinterpret_cast<const void *>(&attn_block_kernel<NCH, I8>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL((attn_block_kernel<NCH, I8>), dim3(m.kv_blocks * c.n_kv_heads), dim3(256), lds, st, m.q16,
                       I8 ? static_cast<const void *>(L.kv8) : static_cast<const void *>(L.kv), L.kvs, m.slots,
                       c.n_heads, c.n_kv_heads, m.sp, m.parts, m.kv_blocks);
    return 0;
}
template <int NCH>
int launch_attn_n(Model &m, LayerW &L, hipStream_t st) {
    return m.kv_i8 ? launch_attn_t<NCH, true>(m, L, st) : launch_attn_t<NCH, false>(m, L, st);
}

int launch_attn(Model &m, LayerW &L, hipStream_t st) {
    switch (m.c.head_dim / 32) {
    case 1: return launch_attn_n<1>(m, L, st);
    case 2: return launch_attn_n<2>(m, L, st);
    case 3: return launch_attn_n<3>(m, L, st);
    case 4: return launch_attn_n<4>(m, L, st);
    case 5: return launch_attn_n<5>(m, L, st);
    case 6: return launch_attn_n<6>(m, L, st);
    case 7: return launch_attn_n<7>(m, L, st);
    default: return launch_attn_n<8>(m, L, st);
    }
}

template <int KW>
int launch_mixout_t(Model &m, LayerW &L, int l, int M, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden;
    MixOutArgs a{};
    a.o = L.o;
    a.act_core = m.act_core;
    a.core_stride = act_halves(L.o.cols);
    a.x = m.x;
    const int64_t ntiles = tiles_rows(H);
    a.o_per = static_cast<int>(tiles_per_wg(ntiles, 8, 1));
    a.router = L.router;
    a.post_norm = L.post_norm;
    a.eps = c.eps;
    a.logits = m.rlogits;
    a.act_h = m.act_h;
    a.act_stride = act_halves(H);
    a.H = H, a.E = c.n_experts, a.E1 = m.E1, a.K = c.top_k;
    a.rs = m.route + l;
    a.ids_out = m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k;
    a.sp = m.sp;
    a.ctr = m.ctr + static_cast<int64_t>(l) * kFlagsPerLayer;
    a.err = m.err;
    a.n_o = static_cast<int>((ntiles + a.o_per - 1) / a.o_per);
    a.n_r = (m.E1 + 3) / 4;
    // (the decode experts' up launch routes the rows itself and clears this launch's flags; a replay of this launch
    // alone keeps its own route workgroup, which clears them)
    a.route_role = up_routes(m, true) ? 0 : 1;
    GV_REQUIRE(a.n_o + a.n_r <= kGdnFlagBase, "mixout: more flags than the launch's share of the layer's");
    GV_REQUIRE(a.n_o + a.n_r == mixout_flags(m), "mixout: the flag count differs from the one the up launch clears");
    const size_t lds = mixout_lds(M, m.E1, a.o_per);
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&mixout_kernel<KW>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(mixout_kernel<KW>, dim3(static_cast<unsigned>(a.n_o + a.n_r + a.route_role)), dim3(512), lds,
                       st, a);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int launch_mixout(Model &m, LayerW &L, int l, int M, int kw, hipStream_t st) {
    if (kw == 16) return launch_mixout_t<16>(m, L, l, M, st);
    if (kw == 8) return launch_mixout_t<8>(m, L, l, M, st);
    return launch_mixout_t<4>(m, L, l, M, st);
}

// One kernel class of layer l (the embedding and lm_head: l ignored) for M rows; the verify step is these in order.
int launch_class(Model &m, int cls, int l, int M, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const int64_t abH = act_halves(H), abC = act_halves(static_cast<int64_t>(nh) * hd);
    LayerW &L = m.layers[static_cast<size_t>(l)];
    // the token mixer's classes of the other kind of layer (attention / Gated DeltaNet) launch nothing
    const bool per_layer = cls != GV_K_EMBED && cls != GV_K_LM_HEAD && cls != GV_K_QUANT;
    const bool gdn_cls = cls >= GV_K_GDN_AB && cls <= GV_K_GDN_NORM;
    const bool attn_cls = cls == GV_K_ROPE || cls == GV_K_ATTN || cls == GV_K_MERGE;
    if (per_layer && (L.gdn ? attn_cls : gdn_cls)) return 0;
    // classes fused into a neighbour launch nothing and take no events
    int mix_kw = 0;
    const bool mixout = mixout_fits(m, M, L.o.cols, mix_kw);
    const bool fused = (cls == GV_K_SWIGLU && m.moe_dec) || (cls == GV_K_ROUTE && m.route_in_router && !m.moe_only) ||
                       ((cls == GV_K_ROUTER || cls == GV_K_ROUTE) && mixout) || (cls == GV_K_GDN_AB && m.fused) ||
                       cls == GV_K_GDN_CONV || cls == GV_K_GDN_NORM;   // (the Gated DeltaNet's: in GV_K_GDN_CORE's)
    if (fused) return 0;
    Tick tk(m, fused ? -2 : cls, st);
    switch (cls) {
    case GV_K_EMBED:
        hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, st, m.embed, m.sp, m.x, m.layers[0].in_norm, c.eps,
                           m.act_h, abH);
        return 0;
    case GV_K_QKV: {   // (a Gated DeltaNet layer: in_proj_qkv | in_proj_z, two globals)
        GemvOut o = qkv_out(m, L);
        if (L.gdn) {
            o.nseg = 2;
            o.seg_end[0] = gdn_conv_dim(c);
            o.seg_end[1] = INT64_MAX;
        }
        o.trace_cls = GV_K_QKV;
        return gemv_q4(L.qkv, m.act_h, abH, M, o, st);
    }
    case GV_K_GDN_AB: {   // the bf16 a / b rows . RMSNorm(x) (the router kernel's arithmetic, bf16_rows' sum order)
        const int E1 = 2 * c.gdn_v_heads, n_dg = (E1 + kRouterRows - 1) / kRouterRows;
        const int wgs = n_dg * ((M + router_tokens(H) - 1) / router_tokens(H));
        if (H <= 2048) {
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&router_kernel<1>), router_lds(H), granted) != 0) return -1;
            hipLaunchKernelGGL(router_kernel<1>, dim3(wgs), dim3(256), router_lds(H), st, L.gdn_ab, E1, H, m.x,
                               L.in_norm, c.eps, m.sp, m.rlogits, nullptr, 0, 0, c.n_experts, c.top_k, m.route + l,
                               nullptr, m.counter, n_dg, -1);
        } else {
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&router_kernel<2>), router_lds(H), granted) != 0) return -1;
            hipLaunchKernelGGL(router_kernel<2>, dim3(wgs), dim3(256), router_lds(H), st, L.gdn_ab, E1, H, m.x,
                               L.in_norm, c.eps, m.sp, m.rlogits, nullptr, 0, 0, c.n_experts, c.top_k, m.route + l,
                               nullptr, m.counter, n_dg, -1);
        }
        GV_CHECK_HIP(hipGetLastError());
        return 0;
    }
    case GV_K_GDN_CORE:   // the conv, the delta rule, the gated norm (and the a / b dots when fused) in one launch
        return gdn_launch(m, L, l, M, !m.fused, st);
    case GV_K_ROPE:
        hipLaunchKernelGGL(qk_rope_kernel, dim3(M, nh + 2 * nkv), dim3(256), 0, st, m.qkv_out, L.qkv.rows, nh, nkv, hd,
                           c.rope_dim / 2, L.q_norm, L.k_norm, c.eps, m.rope_cos, m.rope_sin, m.sp, m.q16, L.kv,
                           L.kv8, L.kvs, m.slots);
        return 0;
    case GV_K_ATTN: {
        return launch_attn(m, L, st);
    }
    case GV_K_MERGE:
        if (hd % 64 == 0)
            hipLaunchKernelGGL(attn_merge64_kernel, dim3(M, nh, hd / 64), dim3(256), 0, st, m.parts, m.qkv_out,
                               L.qkv.rows, nh, hd, m.kv_blocks, m.sp, m.act_core, abC);
        else
            hipLaunchKernelGGL(attn_merge_kernel, dim3(M, nh), dim3(256), 0, st, m.parts, m.qkv_out, L.qkv.rows, nh, hd,
                               m.kv_blocks, m.sp, m.act_core, abC);
        return 0;
    case GV_K_O: {   // the residual add is the product's accumulate
        if (mixout) return launch_mixout(m, L, l, M, mix_kw, st);   // with the router and the route
        GemvOut o = gemv_out(m.x, H, L.o.global, 1);
        o.trace_cls = GV_K_O;
        return gemv_q4(L.o, m.act_core, L.gdn ? act_halves(L.o.cols) : abC, M, o, st);
    }
    case GV_K_ROUTER: {   // workgroups: (router row group, token group), each row's operands by one of them
        const int TG = router_tokens(H);
        // (the MoE block with its routed logits given: only the operands' row groups and the shared expert's)
        const bool shared_only = m.moe_only && m.router_shared_only && (m.E1 - 1) / kRouterRows >= std::min(M, TG);
        const int shared_dg = shared_only ? (m.E1 - 1) / kRouterRows : -1;
        const int n_dg = shared_only ? std::min(M, TG) + 1 : std::max((m.E1 + kRouterRows - 1) / kRouterRows, std::min(M, TG));
        const int wgs = n_dg * ((M + TG - 1) / TG);
        const float *xr = m.moe_only && m.block_h ? m.block_h : m.x;   // (the MoE block's rows as given)
        if (H <= 2048) {
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&router_kernel<1>), router_lds(H), granted) != 0) return -1;
            hipLaunchKernelGGL(router_kernel<1>, dim3(wgs), dim3(256), router_lds(H), st, L.router, m.E1, H, xr,
                               m.moe_only ? nullptr : L.post_norm, c.eps, m.sp, m.rlogits, m.act_h, abH,
                               m.route_in_router && !m.moe_only ? 1 : 0, c.n_experts, c.top_k, m.route + l,
                               m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k, m.counter, n_dg,
                               shared_dg);
        } else {
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&router_kernel<2>), router_lds(H), granted) != 0) return -1;
            hipLaunchKernelGGL(router_kernel<2>, dim3(wgs), dim3(256), router_lds(H), st, L.router, m.E1, H, xr,
                               m.moe_only ? nullptr : L.post_norm, c.eps, m.sp, m.rlogits, m.act_h, abH,
                               m.route_in_router && !m.moe_only ? 1 : 0, c.n_experts, c.top_k, m.route + l,
                               m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k, m.counter, n_dg,
                               shared_dg);
        }
        return 0;
    }
    case GV_K_ROUTE:
        if (m.route_in_router && !m.moe_only) return 0;   // done by the router's last workgroup
        hipLaunchKernelGGL(route_kernel, dim3(1), dim3(1024), 0, st, m.rlogits, c.n_experts, c.top_k, m.sp, m.route + l,
                           m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k);
        return 0;
    case GV_K_MOE_UP:   // with the SwiGLU and its quantization (moe_up_kernel) where the decode variant fits; after
                        // the fused output projection / router launch it also routes the rows
        // (a replay of this launch alone: the slots the step's own route left in the layer's route state)
        return m.moe_dec ? moe_dec(m, L, M, true, up_routes(m, mixout), st) : moe_products(m, L, M, true, st);
    case GV_K_SWIGLU:
        if (m.moe_dec) return 0;
        hipLaunchKernelGGL(swiglu_quant_kernel, dim3(M * (c.top_k + 1)), dim3(256), static_cast<size_t>(c.moe_ff) * 4,
                           st, m.gu_out, c.moe_ff, &m.route[l].n_picks, m.act_m);
        return 0;
    case GV_K_MOE_DOWN:
        return m.moe_dec ? moe_dec(m, L, M, false, false, st) : moe_products(m, L, M, false, st);
    case GV_K_COMBINE: {   // the residual add, then the next layer's input RMSNorm (after the last: the final norm;
                           // after the MTP layer: mtp.norm)
        const bool mtp_layer = l == c.n_layers;
        const float *next_norm = m.moe_only              ? nullptr
                                 : mtp_layer             ? m.mtp_norm
                                 : l + 1 < c.n_layers    ? m.layers[static_cast<size_t>(l) + 1].in_norm
                                                         : m.final_norm;
        // a model with an MTP layer keeps the normalized rows it drafts from: the last layer's (the verify's hidden
        // rows) and the MTP layer's own (a chained draft's)
        float *hout = !m.has_mtp || m.moe_only ? nullptr
                      : mtp_layer             ? m.hbuf + static_cast<int64_t>(c.max_rows) * H
                      : l + 1 == c.n_layers   ? m.hbuf
                                              : nullptr;
        combine_launch(m.y, H, c.top_k, route_mix(m.route + l, m.moe_dec), M, m.x, next_norm, c.eps, m.act_h, abH, st,
                       hout, !m.moe_only);
        return 0;
    }
    case GV_K_LM_HEAD:
        return gemv_q4(m.lm_head, m.act_h, abH, M, gemv_out(m.logits, c.vocab, m.lm_head.global), st);
    default:
        return 0;
    }
}

// (an attention layer skips the GV_K_GDN_* classes, a Gated DeltaNet layer GV_K_ROPE, GV_K_ATTN and GV_K_MERGE)
constexpr int kLayerClassList[] = {GV_K_QKV,    GV_K_GDN_AB, GV_K_GDN_CONV, GV_K_GDN_CORE, GV_K_GDN_NORM,
                                      GV_K_ROPE,   GV_K_ATTN,   GV_K_MERGE,    GV_K_O,        GV_K_ROUTER,
                                      GV_K_ROUTE,  GV_K_MOE_UP, GV_K_SWIGLU,   GV_K_MOE_DOWN, GV_K_COMBINE};

int run_layers(Model &m, int M, hipStream_t st) {
    if (launch_class(m, GV_K_EMBED, 0, M, st) != 0) return -1;
    for (int l = 0; l < m.c.n_layers; ++l)
        for (int cls : kLayerClassList)
            if (launch_class(m, cls, l, M, st) != 0) return -1;
    if (launch_class(m, GV_K_LM_HEAD, 0, M, st) != 0) return -1;
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// A fused launch's bounded wait that ran out (a producer never signalled: a bug, reported rather than hung on): the
// flag read back after the stream's work; the step's results are then not to be trusted.
int check_wait_flag(Model &m, hipStream_t st) {
    int flag = 0;
    GV_CHECK_HIP(hipMemcpyAsync(&flag, m.err, 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    GV_REQUIRE(flag == 0, "verify: a fused launch's wait for its producers ran out (the step's results are invalid)");
    return 0;
}

// the verify step's launches: replayed from the row count's graph when there is one (captured on the second step of
// that row count, so the first runs the launches directly and sets every kernel's attributes)
int run_step(Model &m, int M, hipStream_t st) {
    if (!m.use_graphs || m.timed_class >= 0 || !m.seen[M]) {
        m.seen[M] = true;
        return run_layers(m, M, st);
    }
    hipGraphExec_t &ge = m.graphs[M];
    if (!ge) {
        hipGraph_t graph = nullptr;
        GV_CHECK_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        const int rc = run_layers(m, M, st);
        const hipError_t e = hipStreamEndCapture(st, &graph);
        if (rc != 0 || e != hipSuccess || !graph) {
            if (graph) (void)hipGraphDestroy(graph);
            set_error(std::string("verify: graph capture failed: ") + (rc != 0 ? last_error() : hipGetErrorString(e)));
            return -1;
        }
        const hipError_t ie = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        GV_REQUIRE(ie == hipSuccess, std::string("verify: graph instantiate failed: ") + hipGetErrorString(ie));
    }
    GV_CHECK_HIP(hipGraphLaunch(ge, st));
    return 0;
}

// the prefill buffers for M rows (kept for later calls; regrown when M is larger)
int prefill_alloc(Model &m, int M) {
    Prefill &pf = m.pf;
    if (pf.cap >= M) return 0;
    for (void *p : pf.allocs) (void)hipFree(p);
    pf.allocs.clear();
    const int cap = (M + 511) / 512 * 512;
    const auto &c = m.c;
    const int64_t H = c.hidden, F = c.moe_ff, E1 = m.E1, K = c.top_k;
    pf.max_picks = cap * (c.top_k + 1);
    pf.max_slots = static_cast<int>(E1 + pf.max_picks / 32 + 1);
    bool ok = true;
    auto get = [&](size_t bytes) -> void * {
        void *p = nullptr;
        if (!ok || hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
            ok = false;
            return nullptr;
        }
        pf.allocs.push_back(p);
        return p;
    };
    pf.h = static_cast<float *>(get(cap * H * 4));
    pf.logits = static_cast<float *>(get(cap * E1 * 4));
    pf.gate = static_cast<float *>(get(cap * 4));
    pf.w = static_cast<float *>(get(cap * K * 4));
    pf.ids = static_cast<int *>(get(cap * K * 4));
    pf.cnt = static_cast<int *>(get(E1 * 4));
    pf.start = static_cast<int *>(get(E1 * 4));
    pf.n_slots = static_cast<int *>(get(4));
    pf.n_picks = static_cast<int *>(get(4));
    pf.slot_expert = static_cast<int *>(get(static_cast<size_t>(pf.max_slots) * 4));
    pf.slot_start = static_cast<int *>(get(static_cast<size_t>(pf.max_slots) * 4));
    pf.slot_count = static_cast<int *>(get(static_cast<size_t>(pf.max_slots) * 4));
    pf.pick_token = static_cast<int *>(get(static_cast<size_t>(pf.max_picks) * 4));
    pf.pick_of = static_cast<int *>(get(cap * (K + 1) * 4));
    pf.act = static_cast<_Float16 *>(get(cap * act_bytes(H)));
    pf.gu = static_cast<float *>(get(static_cast<size_t>(pf.max_picks) * 2 * F * 4));
    pf.act_m = static_cast<_Float16 *>(get(static_cast<size_t>(pf.max_picks) * act_bytes(F)));
    pf.y = static_cast<float *>(get(static_cast<size_t>(pf.max_picks) * H * 4));
    pf.out = static_cast<float *>(get(cap * H * 4));
    GV_REQUIRE(ok, "prefill MoE: out of device memory");
    pf.cap = cap;
    return 0;
}

// The MoE block of layer `layer` on the M rows in pf.h with the routed logits in pf.logits [M][E + 1] (column E
// filled here: the shared expert's gate logit): route each row, group the picks by expert (runs of at most 32),
// the experts' products, SwiGLU, down, and the combine into pf.out (no residual).
int moe_prefill(Model &m, int layer, int M, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden, E = c.n_experts, K = c.top_k, F = c.moe_ff;
    Prefill &pf = m.pf;
    LayerW &L = m.layers[static_cast<size_t>(layer)];
    if (m.fused && H <= kPrefillFrontMaxH) {   // two launches (prefill.hip), the same outputs as the five below
        if (prefill_route(pf.logits, M, E, K, pf.ids, pf.w, st) != 0 ||
            prefill_rest(L.router + static_cast<int64_t>(E) * H, H, pf.h, M, E, K, pf.logits, pf.gate, pf.act,
                         act_halves(H), pf.ids, pf.start, pf.n_slots, pf.slot_expert, pf.slot_start, pf.slot_count,
                         pf.n_picks, pf.pick_token, pf.pick_of, st) != 0)
            return -1;
    } else {
        if (quantize_act(pf.h, H, M, H, nullptr, 0.0f, pf.act, act_halves(H), nullptr, 0, st) != 0) return -1;
        const int wg4 = (M + 3) / 4;
        {
            const size_t lds = static_cast<size_t>(5) * H * 4;   // the gate row and the 4 waves' rows as fp32
            static int granted = 0;
            if (lds_grant(reinterpret_cast<const void *>(&gate_rows_kernel), lds, granted) != 0) return -1;
            hipLaunchKernelGGL(gate_rows_kernel, dim3(wg4), dim3(256), lds, st, L.router + static_cast<int64_t>(E) * H,
                               H, pf.h, M, pf.logits, m.E1);
        }
        hipLaunchKernelGGL(route_rows_kernel, dim3(wg4), dim3(256), 0, st, pf.logits, E, K, M, pf.ids, pf.w, pf.gate);
        hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, st, pf.ids, M, K, E, pf.start, pf.n_slots,
                           pf.slot_expert, pf.slot_start, pf.slot_count, pf.n_picks);
        hipLaunchKernelGGL(fill_picks_kernel, dim3(m.E1), dim3(256), 0, st, pf.ids, M, K, E, pf.start, pf.pick_token,
                           pf.pick_of);
        GV_CHECK_HIP(hipGetLastError());
    }
    const Slots sl{pf.n_slots, pf.slot_expert, pf.slot_start, pf.slot_count, pf.pick_token, pf.n_picks, nullptr,
                   nullptr};
    const int picks = M * (K + 1);
    // gate|up with the SwiGLU and its quantization in the launch (matched tile pairs), then down
    if (moe_run(m, L, true, 32, pf.act, pf.gu, sl, pf.gu, pf.max_slots, picks, st, pf.act_m) != 0) return -1;
    if (moe_run(m, L, false, 32, pf.act_m, pf.gu, sl, pf.y, pf.max_slots, picks, st) != 0) return -1;
    combine_launch(pf.y, H, K, MixView{pf.gate, pf.w, pf.pick_of}, M, pf.out, nullptr, 0.0f, nullptr, 0, st, nullptr,
                   false);
    GV_CHECK_HIP(hipGetLastError());
    pf.M = M;
    return 0;
}

void *dalloc(Model &m, size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
    m.allocs.push_back(p);
    return p;
}

bool alloc_q4(Model &m, Q4 &q, int64_t rows, int64_t cols) {
    auto *p = static_cast<uint8_t *>(dalloc(m, q4_code_bytes(rows, cols) + q4_scale_bytes(rows, cols)));
    if (!p) return false;
    q.codes = p;
    q.scales = p + q4_code_bytes(rows, cols);
    q.rows = rows;
    q.cols = cols;
    return true;
}

// the Gated DeltaNet layers' slots of a step: the rows start from the base, their states go to the other set
void set_gdn_slots(const Model &m, StepParams &sp) {
    sp.gdn_base = m.gdn_base;
    sp.gdn_wset = m.gdn_base < m.c.max_rows ? m.c.max_rows : 0;
}

int64_t qkv_rows(const gv_model_config &c) {
    return static_cast<int64_t>(c.n_heads) * 2 * c.head_dim + 2 * static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
}

}  // namespace

int run_class(Model &m, int cls, int l, int M, hipStream_t st) { return launch_class(m, cls, l, M, st); }
GV_ACT_MODE_SETTER(act_mode_set_model)
const int *layer_classes(int &count) {
    count = static_cast<int>(sizeof(kLayerClassList) / sizeof(kLayerClassList[0]));
    return kLayerClassList;
}

}  // namespace gv

using namespace gv;

struct gv_model {
    Model m;
    std::vector<uint8_t *> staging;   // device staging, freed at the end of the call that made it
};

Model &gv::model_of(gv_model *g) { return g->m; }

namespace {
void put_err(char *err, int err_len, const std::string &msg) {
    if (err && err_len > 0) {
        std::strncpy(err, msg.c_str(), static_cast<size_t>(err_len) - 1);
        err[err_len - 1] = '\0';
    }
}

// a pack-layout q4 matrix (host or device bytes) into a device-layout allocation
int upload_q4(const void *pack, bool on_device, int64_t rows, int64_t cols, uint8_t *codes, uint8_t *scales,
              float global, Q4 &out) {
    const size_t bytes = static_cast<size_t>(rows) * static_cast<size_t>(cols / 16) * 9;
    const uint8_t *src = static_cast<const uint8_t *>(pack);
    void *tmp = nullptr;
    if (!on_device) {
        GV_CHECK_HIP(hipMalloc(&tmp, bytes));
        GV_CHECK_HIP(hipMemcpyAsync(tmp, pack, bytes, hipMemcpyHostToDevice, stream()));
        src = static_cast<const uint8_t *>(tmp);
    }
    const int rc = q4_from_pack(src, rows, cols, global, codes, scales, out, stream());
    if (tmp) {
        (void)hipStreamSynchronize(stream());
        (void)hipFree(tmp);
    }
    return rc;
}
}  // namespace

extern "C" {

gv_model *gv_model_create(const gv_model_config *cfg, char *err, int err_len) {
    if (ensure_init() != 0) {
        put_err(err, err_len, last_error());
        return nullptr;
    }
    const gv_model_config c = *cfg;
    Model *made = nullptr;   // once set, a failure frees what it allocated
    auto fail = [&](const std::string &msg) -> gv_model * {
        if (made) {
            mtp_release(*made);
            for (void *p : made->allocs) (void)hipFree(p);
            made->allocs.clear();
        }
        put_err(err, err_len, msg);
        set_error(msg);
        return nullptr;
    };
    if (c.hidden <= 0 || c.hidden % 128 != 0 || c.hidden > kMaxActCols)
        return fail("hidden must be a positive multiple of 128, at most 16384");
    if (c.moe_ff > kMaxActCols) return fail("moe_ff at most 16384");
    if (c.moe_ff <= 0 || c.moe_ff % 128 != 0 || c.shared_ff != c.moe_ff)
        return fail("moe_ff must be a positive multiple of 128 and shared_ff equal to it");
    if (c.head_dim <= 0 || c.head_dim > 256 || c.head_dim % 32 != 0 || c.rope_dim > c.head_dim || c.rope_dim % 2)
        return fail("head_dim must be a multiple of 32 up to 256, rope_dim even and <= head_dim");
    if ((c.max_ctx + kAttnBlock - 1) / kAttnBlock > 1024) return fail("max_ctx at most 65536 positions");
    if (c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads != 0 || (c.n_heads * c.head_dim) % 128 != 0)
        return fail("n_heads must be a multiple of n_kv_heads, n_heads x head_dim a multiple of 128");
    if (c.n_experts <= 0 || c.n_experts > 256 || c.top_k <= 0 || c.top_k > 16 || c.top_k > c.n_experts)
        return fail("1 <= top_k <= 16, top_k <= n_experts <= 256");
    if (c.max_rows <= 0 || c.max_rows > kMaxRows) return fail("max_rows must be 1..32");
    if (c.mtp != 0 && (c.mtp != 1 || c.hidden > 8192)) return fail("mtp must be 0 or 1 (an MTP layer: hidden at most 8192)");
    if (c.exact != 0 && (c.exact != 1 || c.kv_int8 != 0)) return fail("exact must be 0 or 1, and the exact path takes no int8 cache");
    if (c.vocab <= 0 || c.n_layers <= 0 || c.max_ctx <= c.max_rows) return fail("vocab, n_layers, max_ctx");
    {
        std::string why;
        if (!gdn_shape_ok(c, why)) return fail(why);
        for (int l = c.n_layers; l < 256; ++l)
            if (c.gdn_layers[l] != 0) return fail("gdn_layers marks a layer past n_layers");
        if (c.n_layers > 256 && c.gdn_v_heads > 0) return fail("Gated DeltaNet models take at most 256 layers");
    }
    {
        int waves, kw;
        const int ntt = c.max_rows <= 16 ? 1 : 2;
        if (!mfma_split(c.hidden, ntt, waves, kw) || !mfma_split(c.moe_ff, ntt, waves, kw))
            return fail("the expert products take hidden and moe_ff up to 4096 (2048 when max_rows > 16)");
    }
    auto g = std::make_unique<gv_model>();
    Model &m = g->m;
    made = &m;
    m.c = c;
    m.E1 = c.n_experts + 1;
    const int64_t H = c.hidden, F = c.moe_ff, V = c.vocab, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    m.gu_code_stride = q4_code_bytes(2 * F, H);
    m.gu_scale_stride = q4_scale_bytes(2 * F, H);
    m.dn_code_stride = q4_code_bytes(H, F);
    m.dn_scale_stride = q4_scale_bytes(H, F);
    bool ok = alloc_q4(m, m.embed, V, H) && alloc_q4(m, m.lm_head, V, H);
    ok = ok && (m.final_norm = static_cast<float *>(dalloc(m, H * 4)));
    m.slots = (static_cast<int64_t>(c.max_ctx) + kAttnBlock - 1) / kAttnBlock * kAttnBlock;
    const size_t kv_layer = 2 * static_cast<size_t>(nkv) * m.slots * hd;   // values a layer
    m.kv_i8 = c.kv_int8 != 0;
    m.kv_layer_bytes = m.kv_i8 ? kv_layer + 2 * static_cast<size_t>(nkv) * m.slots * 4 : kv_layer * 2;
    m.kv_layer_bytes = (m.kv_layer_bytes + 255) / 256 * 256;
    // the layers: the main ones, then the MTP layer's (index n_layers: an attention layer, its KV after theirs)
    m.has_mtp = c.mtp != 0;
    const int NL = c.n_layers + (m.has_mtp ? 1 : 0);
    m.kv_all = static_cast<_Float16 *>(dalloc(m, static_cast<size_t>(NL) * m.kv_layer_bytes));
    ok = ok && m.kv_all;
    m.layers.resize(static_cast<size_t>(NL));
    const int64_t gconv = gdn_conv_dim(c), gvd = static_cast<int64_t>(c.gdn_v_heads) * c.gdn_v_dim;
    for (int l = 0; ok && l < NL; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        L.gdn = c.gdn_v_heads > 0 && l < c.n_layers && l < 256 && c.gdn_layers[l] != 0;
        if (L.gdn) {   // in_proj_qkv | in_proj_z, out_proj, the bf16 a / b rows, the small tensors, the state slots
            const int64_t nv = c.gdn_v_heads, K = c.conv_kernel, Mx2 = 2 * static_cast<int64_t>(c.max_rows);
            ok = alloc_q4(m, L.qkv, gconv + gvd, H) && alloc_q4(m, L.o, H, gvd);
            ok = ok && (L.gdn_ab = static_cast<uint16_t *>(dalloc(m, static_cast<size_t>(2 * nv * H) * 2)));
            auto *gf = ok ? static_cast<float *>(dalloc(m, static_cast<size_t>(2 * nv + gconv * K + c.gdn_v_dim) * 4))
                          : nullptr;
            ok = ok && gf;
            if (ok) L.A_log = gf, L.dt_bias = gf + nv, L.conv_w = gf + 2 * nv, L.gnorm = gf + 2 * nv + gconv * K;
            const size_t sb = static_cast<size_t>(Mx2 * gdn_s_floats(c)) * 4, cb = static_cast<size_t>(Mx2 * gdn_c_floats(c)) * 4;
            ok = ok && (L.s_slots = static_cast<float *>(dalloc(m, sb))) && hipMemset(L.s_slots, 0, sb) == hipSuccess;
            ok = ok && (L.c_slots = static_cast<float *>(dalloc(m, cb))) && hipMemset(L.c_slots, 0, cb) == hipSuccess;
        } else {
            ok = alloc_q4(m, L.qkv, qkv_rows(c), H) && alloc_q4(m, L.o, H, nh * hd);
        }
        auto *f = ok ? static_cast<float *>(dalloc(m, (2 * H + 2 * hd) * 4)) : nullptr;
        ok = ok && f;
        if (!ok) break;
        L.in_norm = f, L.post_norm = f + H, L.q_norm = f + 2 * H, L.k_norm = f + 2 * H + hd;
        L.router = static_cast<uint16_t *>(dalloc(m, static_cast<size_t>(m.E1) * H * 2));
        auto *gu = static_cast<uint8_t *>(dalloc(m, (m.gu_code_stride + m.gu_scale_stride) * m.E1));
        auto *dn = static_cast<uint8_t *>(dalloc(m, (m.dn_code_stride + m.dn_scale_stride) * m.E1));
        L.expert_globals = static_cast<float *>(dalloc(m, static_cast<size_t>(m.E1) * 3 * 4));
        ok = L.router && gu && dn && L.expert_globals;
        if (!ok) break;
        L.gu_codes = gu, L.gu_scales = gu + m.gu_code_stride * m.E1;
        L.dn_codes = dn, L.dn_scales = dn + m.dn_code_stride * m.E1;
        uint8_t *kb = reinterpret_cast<uint8_t *>(m.kv_all) + static_cast<size_t>(l) * m.kv_layer_bytes;
        if (m.kv_i8) {
            L.kv8 = reinterpret_cast<int8_t *>(kb);
            L.kvs = reinterpret_cast<float *>(kb + kv_layer);
        } else {
            L.kv = reinterpret_cast<_Float16 *>(kb);
        }
    }
    for (int l = 0; l < NL; ++l) (m.layers[static_cast<size_t>(l)].gdn ? m.gdn_layers : m.attn_layers).push_back(l);
    ok = ok && (m.attn_index = static_cast<int *>(dalloc(m, std::max<size_t>(1, m.attn_layers.size()) * 4)));
    ok = ok && (m.attn_layers.empty() || hipMemcpy(m.attn_index, m.attn_layers.data(), m.attn_layers.size() * 4,
                                                   hipMemcpyHostToDevice) == hipSuccess);
    const int Mx = c.max_rows, K = c.top_k;
    m.max_slots = moe_slots_bound(c.n_experts, K, Mx);
    if (m.max_slots > kRouteSlots) return fail("gv_model_create: too many expert slots for the route state");
    m.max_picks = Mx * (K + 1);
    m.kv_blocks = (c.max_ctx + kAttnBlock - 1) / kAttnBlock;
    ok = ok && (m.sp = static_cast<StepParams *>(dalloc(m, sizeof(StepParams))));
    ok = ok && (m.route = static_cast<RouteState *>(dalloc(m, sizeof(RouteState) * NL)));
    ok = ok && (m.counter = static_cast<int *>(dalloc(m, 64)));
    ok = ok && hipMemset(m.counter, 0, 64) == hipSuccess;
    const size_t ctr_bytes = static_cast<size_t>(NL) * kFlagsPerLayer * 4 + 256;   // the fused launches' flags, err
    ok = ok && (m.ctr = static_cast<int *>(dalloc(m, ctr_bytes)));
    ok = ok && hipMemset(m.ctr, 0, ctr_bytes) == hipSuccess;
    if (ok) m.err = m.ctr + static_cast<size_t>(NL) * kFlagsPerLayer;
    {
        int kwu, kwd, waves;
        m.moe_dec = moe_dec_shape(c, kwu, kwd, waves);
    }
    {   // the buffers one step's phases exchange, in one arena (one allocation, 256-byte aligned pieces)
        const size_t sizes[] = {static_cast<size_t>(Mx) * H * 4,
                                static_cast<size_t>(Mx) * std::max(qkv_rows(c), gconv + gvd) * 4,
                                static_cast<size_t>(Mx) * std::max(m.E1, 2 * c.gdn_v_heads) * 4,
                                static_cast<size_t>(Mx) * nh * m.kv_blocks * (hd + 2) * 4,
                                static_cast<size_t>(m.max_picks) * H * 4,
                                static_cast<size_t>(Mx) * V * 4,
                                static_cast<size_t>(Mx) * act_bytes(H),
                                static_cast<size_t>(Mx) * act_bytes(std::max(nh * hd, gvd)),
                                static_cast<size_t>(m.max_picks) * act_bytes(F),
                                static_cast<size_t>(Mx) * gvd * 4};
        size_t offs[10], tot = 0;
        for (int i = 0; i < 10; ++i) {
            offs[i] = tot;
            tot += (sizes[i] + 255) / 256 * 256;
        }
        auto *ar = static_cast<uint8_t *>(dalloc(m, tot));
        ok = ok && ar && tot < 0x7FFFFF00u;
        if (ok) {
            m.arena = ar;
            m.arena_bytes = tot;
            m.x = reinterpret_cast<float *>(ar + offs[0]);
            m.qkv_out = reinterpret_cast<float *>(ar + offs[1]);
            m.rlogits = reinterpret_cast<float *>(ar + offs[2]);
            m.parts = reinterpret_cast<float *>(ar + offs[3]);
            m.y = reinterpret_cast<float *>(ar + offs[4]);
            m.logits = reinterpret_cast<float *>(ar + offs[5]);
            m.act_h = reinterpret_cast<_Float16 *>(ar + offs[6]);
            m.act_core = reinterpret_cast<_Float16 *>(ar + offs[7]);
            m.act_m = reinterpret_cast<_Float16 *>(ar + offs[8]);
            m.gdn_core = gvd > 0 ? reinterpret_cast<float *>(ar + offs[9]) : nullptr;
        }
    }
    ok = ok && (m.q16 = static_cast<_Float16 *>(dalloc(m, 2 * Mx * nh * hd * 2)));
    ok = ok && (m.gu_out = static_cast<float *>(dalloc(m, static_cast<size_t>(m.max_picks) * 2 * F * 4)));
    ok = ok && (m.route_ids = static_cast<int32_t *>(dalloc(m, static_cast<size_t>(NL) * Mx * K * 4)));
    ok = ok && (!m.has_mtp || mtp_alloc(m) == 0);
    const int half = c.rope_dim / 2;
    const int npos = c.max_ctx + kMaxRows;
    ok = ok && (m.rope_cos = static_cast<float *>(dalloc(m, static_cast<size_t>(npos) * std::max(1, half) * 4)));
    ok = ok && (m.rope_sin = static_cast<float *>(dalloc(m, static_cast<size_t>(npos) * std::max(1, half) * 4)));
    if (!ok) return fail("gv_model_create: out of device memory");
    // the rotary table on the host with the reference's float functions (model.cpp:739-740, :3719-3723)
    std::vector<float> inv(static_cast<size_t>(half)), cs(static_cast<size_t>(npos) * half), sn(cs.size());
    for (int i = 0; i < half; ++i)
        inv[static_cast<size_t>(i)] = 1.0f / std::pow(c.rope_theta, static_cast<float>(2 * i) / static_cast<float>(c.rope_dim));
    for (int p = 0; p < npos; ++p)
        for (int i = 0; i < half; ++i) {
            const float f = static_cast<float>(p) * inv[static_cast<size_t>(i)];
            cs[static_cast<size_t>(p) * half + i] = std::cos(f);
            sn[static_cast<size_t>(p) * half + i] = std::sin(f);
        }
    if (half > 0 &&
        (hipMemcpy(m.rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
         hipMemcpy(m.rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess))
        return fail("gv_model_create: rope table copy failed");
    if (hipMemset(m.kv_all, 0, static_cast<size_t>(NL) * m.kv_layer_bytes) != hipSuccess)
        return fail("gv_model_create: memset failed");
    return g.release();
}

void gv_model_free(gv_model *g) {
    if (!g) return;
    (void)hipStreamSynchronize(stream());
    for (auto &ge : g->m.graphs)
        if (ge) (void)hipGraphExecDestroy(ge);
    mtp_release(g->m);
    for (void *p : g->m.allocs) (void)hipFree(p);
    for (void *p : g->m.pf.allocs) (void)hipFree(p);
    if (g->m.trace) {   // the kernels stop stamping before the buffer goes
        uint64_t *none = nullptr;
        (void)hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &none, sizeof none);
        (void)trace_set_q4(nullptr);
        (void)trace_set_gdn(nullptr);
        (void)hipFree(g->m.trace);
    }
    delete g;
}

int gv_model_adopt(gv_model *g, int kind, int layer, int expert, const void *data, int64_t bytes,
                   const float *globals) {
    GV_REQUIRE(g && data, "gv_model_adopt: null pointer");
    Model &m = g->m;
    const auto &c = m.c;
    const int64_t H = c.hidden, F = c.moe_ff, V = c.vocab, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const bool mtp_kind = kind >= GV_MTP_FC && kind <= GV_MTP_PRE_H;
    GV_REQUIRE(!mtp_kind || m.has_mtp, "gv_model_adopt: an MTP tensor for a model without an MTP layer");
    const bool per_layer = kind != GV_EMBED && kind != GV_LM_HEAD && kind != GV_FINAL_NORM && !mtp_kind;
    GV_REQUIRE(!per_layer || (layer >= 0 && layer < static_cast<int>(m.layers.size())),
               "gv_model_adopt: no such layer (n_layers: the MTP layer's)");
    LayerW *L = per_layer ? &m.layers[static_cast<size_t>(layer)] : nullptr;
    auto q4_size = [](int64_t r, int64_t cc) { return r * (cc / 16) * 9; };
    auto copy = [&](void *dst, int64_t want) -> int {
        GV_REQUIRE(bytes == want, "gv_model_adopt: wrong size for this tensor");
        GV_CHECK_HIP(hipMemcpy(dst, data, static_cast<size_t>(bytes), hipMemcpyHostToDevice));
        return 0;
    };
    const bool gdn_kind = kind >= GV_GDN_QKV && kind <= GV_GDN_S;
    const bool attn_kind = kind == GV_QKV || kind == GV_O || kind == GV_Q_NORM || kind == GV_K_NORM || kind == GV_KV ||
                           kind == GV_KV_I8;
    GV_REQUIRE(!gdn_kind || L->gdn, "gv_model_adopt: a Gated DeltaNet tensor for an attention layer");
    GV_REQUIRE(!attn_kind || !L->gdn, "gv_model_adopt: an attention tensor for a Gated DeltaNet layer");
    const int64_t nv = c.gdn_v_heads, gconv = gdn_conv_dim(c), gvd = nv * c.gdn_v_dim;
    switch (kind) {
    case GV_GDN_QKV:
    case GV_GDN_Z: {   // the two parts of the layer's qkv matrix (whole 16-row tiles each: conv_dim is a multiple of 64)
        const bool z = kind == GV_GDN_Z;
        const int64_t rows = z ? gvd : gconv;
        GV_REQUIRE(globals && bytes == q4_size(rows, H), "gv_model_adopt: in_proj_qkv / in_proj_z size");
        Q4 tmp;
        const size_t co = z ? q4_code_bytes(gconv, H) : 0, so = z ? q4_scale_bytes(gconv, H) : 0;
        if (upload_q4(data, false, rows, H, const_cast<uint8_t *>(L->qkv.codes) + co,
                      const_cast<uint8_t *>(L->qkv.scales) + so, 1.0f, tmp) != 0)
            return -1;
        (z ? L->g_k : L->g_q) = globals[0];
        return 0;
    }
    case GV_GDN_OUT:
        GV_REQUIRE(globals && bytes == q4_size(H, gvd), "gv_model_adopt: out_proj size");
        return upload_q4(data, false, H, gvd, const_cast<uint8_t *>(L->o.codes), const_cast<uint8_t *>(L->o.scales),
                         globals[0], L->o);
    case GV_GDN_A: return copy(L->gdn_ab, nv * H * 2);
    case GV_GDN_B: return copy(L->gdn_ab + nv * H, nv * H * 2);
    case GV_GDN_ALOG: return copy(L->A_log, nv * 4);
    case GV_GDN_DTB: return copy(L->dt_bias, nv * 4);
    case GV_GDN_CONV: return copy(L->conv_w, gconv * c.conv_kernel * 4);
    case GV_GDN_NORM: return copy(L->gnorm, static_cast<int64_t>(c.gdn_v_dim) * 4);
    case GV_GDN_CONV_ST:   // the states go to the base slot: the next verify's rows start from them
        GV_REQUIRE(bytes == gdn_c_floats(c) * 4, "gv_model_adopt: conv state size");
        return gdn_put_state(m, *L, m.gdn_base, static_cast<const float *>(data), nullptr);
    case GV_GDN_S:
        GV_REQUIRE(bytes == gdn_s_floats(c) * 4, "gv_model_adopt: recurrent state size");
        return gdn_put_state(m, *L, m.gdn_base, nullptr, static_cast<const float *>(data));
    case GV_EMBED:
    case GV_LM_HEAD: {
        GV_REQUIRE(globals && bytes == q4_size(V, H), "gv_model_adopt: embed / lm_head size");
        Q4 &q = kind == GV_EMBED ? m.embed : m.lm_head;
        return upload_q4(data, false, V, H, const_cast<uint8_t *>(q.codes), const_cast<uint8_t *>(q.scales),
                         globals[0], q);
    }
    case GV_FINAL_NORM: return copy(m.final_norm, H * 4);
    case GV_MTP_FC:
        GV_REQUIRE(globals && bytes == q4_size(H, 2 * H), "gv_model_adopt: mtp.fc size");
        return upload_q4(data, false, H, 2 * H, const_cast<uint8_t *>(m.mtp_fc.codes),
                         const_cast<uint8_t *>(m.mtp_fc.scales), globals[0], m.mtp_fc);
    case GV_MTP_NORM: return copy(m.mtp_norm, H * 4);
    case GV_MTP_PRE_E: return copy(m.mtp_pre_e, H * 4);
    case GV_MTP_PRE_H: return copy(m.mtp_pre_h, H * 4);
    case GV_IN_NORM: return copy(L->in_norm, H * 4);
    case GV_POST_NORM: return copy(L->post_norm, H * 4);
    case GV_Q_NORM: return copy(L->q_norm, hd * 4);
    case GV_K_NORM: return copy(L->k_norm, hd * 4);
    case GV_QKV: {
        GV_REQUIRE(globals && bytes == q4_size(qkv_rows(c), H), "gv_model_adopt: qkv size");
        L->g_q = globals[0], L->g_k = globals[1], L->g_v = globals[2];
        return upload_q4(data, false, qkv_rows(c), H, const_cast<uint8_t *>(L->qkv.codes),
                         const_cast<uint8_t *>(L->qkv.scales), 1.0f, L->qkv);
    }
    case GV_O: {
        GV_REQUIRE(globals && bytes == q4_size(H, nh * hd), "gv_model_adopt: o size");
        return upload_q4(data, false, H, nh * hd, const_cast<uint8_t *>(L->o.codes), const_cast<uint8_t *>(L->o.scales),
                         globals[0], L->o);
    }
    case GV_ROUTER: return copy(L->router, static_cast<int64_t>(c.n_experts) * H * 2);
    case GV_SHARED_GATE: return copy(L->router + static_cast<size_t>(c.n_experts) * H, H * 2);
    case GV_EXPERT:
    case GV_SHARED_EXPERT: {
        const int e = kind == GV_EXPERT ? expert : c.n_experts;
        GV_REQUIRE(e >= 0 && e <= c.n_experts, "gv_model_adopt: no such expert");
        GV_REQUIRE(globals && bytes == q4_size(2 * F, H) + q4_size(H, F), "gv_model_adopt: expert block size");
        const float gl[3] = {globals[0], kind == GV_EXPERT ? globals[0] : globals[1],
                             kind == GV_EXPERT ? globals[1] : globals[2]};
        Q4 tmp;
        if (upload_q4(data, false, 2 * F, H, L->gu_codes + e * m.gu_code_stride, L->gu_scales + e * m.gu_scale_stride,
                      gl[0], tmp) != 0)
            return -1;
        if (upload_q4(static_cast<const uint8_t *>(data) + q4_size(2 * F, H), false, H, F,
                      L->dn_codes + e * m.dn_code_stride, L->dn_scales + e * m.dn_scale_stride, gl[2], tmp) != 0)
            return -1;
        GV_CHECK_HIP(hipMemcpy(L->expert_globals + e * 3, gl, 12, hipMemcpyHostToDevice));
        return 0;
    }
    case GV_KV: {
        const int64_t kv_row = nkv * hd;
        GV_REQUIRE(bytes % (2 * kv_row * 2) == 0 && bytes / (2 * kv_row * 2) <= c.max_ctx, "gv_model_adopt: kv size");
        const int64_t n = bytes / (2 * kv_row * 2);
        if (n == 0) return 0;   // an empty context: nothing to convert
        std::vector<float> f(static_cast<size_t>(2 * n * kv_row));
        const auto *hsrc = static_cast<const uint16_t *>(data);
        for (size_t i = 0; i < f.size(); ++i) f[i] = static_cast<float>(__builtin_bit_cast(_Float16, hsrc[i]));
        float *dsrc = nullptr;
        GV_CHECK_HIP(hipMalloc(&dsrc, f.size() * 4 + 4));
        GV_CHECK_HIP(hipMemcpy(dsrc, f.data(), f.size() * 4, hipMemcpyHostToDevice));
        if (m.kv_i8)   // an int8 cache quantizes the rows (quant_kv_row)
            hipLaunchKernelGGL(kv8_from_rows_kernel, dim3(static_cast<unsigned>(2 * n * nkv)), dim3(256), 0, stream(),
                               dsrc, static_cast<int>(n), static_cast<int>(nkv), static_cast<int>(hd), m.slots, L->kv8,
                               L->kvs);
        else
            hipLaunchKernelGGL(kv_from_rows_kernel, dim3(static_cast<unsigned>((f.size() + 255) / 256)), dim3(256), 0,
                               stream(), dsrc, static_cast<int>(n), static_cast<int>(nkv), static_cast<int>(hd), m.slots,
                               L->kv);
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipStreamSynchronize(stream()));
        GV_CHECK_HIP(hipFree(dsrc));
        return 0;
    }
    case GV_KV_I8: {   // the reference's int8 rows and scales, as they are
        GV_REQUIRE(m.kv_i8, "gv_model_adopt: GV_KV_I8 needs a model made with kv_int8");
        const int64_t kv_row = nkv * hd, per = 2 * (kv_row + nkv * 4);   // bytes a position
        GV_REQUIRE(bytes % per == 0 && bytes / per <= c.max_ctx, "gv_model_adopt: int8 kv size");
        const int64_t n = bytes / per;
        if (n == 0) return 0;
        void *dsrc = nullptr;
        GV_CHECK_HIP(hipMalloc(&dsrc, static_cast<size_t>(bytes)));
        GV_CHECK_HIP(hipMemcpy(dsrc, data, static_cast<size_t>(bytes), hipMemcpyHostToDevice));
        const auto *q = static_cast<const int8_t *>(dsrc);
        const auto *sc = reinterpret_cast<const float *>(q + 2 * n * kv_row);
        hipLaunchKernelGGL(kv8_copy_kernel, dim3(static_cast<unsigned>((2 * n * kv_row + 255) / 256)), dim3(256), 0,
                           stream(), q, sc, static_cast<int>(n), static_cast<int>(nkv), static_cast<int>(hd), m.slots,
                           L->kv8, L->kvs);
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipStreamSynchronize(stream()));
        GV_CHECK_HIP(hipFree(dsrc));
        return 0;
    }
    default: set_error("gv_model_adopt: unknown tensor kind"); return -1;
    }
}

int gv_model_randomize(gv_model *g, uint64_t seed, float sigma, float router_sigma, int ctx) {
    GV_REQUIRE(g, "gv_model_randomize: null model");
    Model &m = g->m;
    const auto &c = m.c;
    GV_REQUIRE(ctx >= 0 && ctx + c.max_rows <= c.max_ctx, "gv_model_randomize: ctx too large");
    const int64_t H = c.hidden, F = c.moe_ff, V = c.vocab, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const int64_t kv_row = nkv * hd;
    hipStream_t st = stream();
    const int64_t biggest = std::max<int64_t>({V * H, qkv_rows(c) * H, 2 * F * H, 2 * static_cast<int64_t>(ctx) * kv_row,
                                               static_cast<int64_t>(m.E1) * H, (gdn_conv_dim(c) + 2 * c.gdn_v_heads *
                                               static_cast<int64_t>(c.gdn_v_dim)) * H, gdn_s_floats(c),
                                               gdn_c_floats(c) * c.conv_kernel});
    float *wf = nullptr;
    uint8_t *pack = nullptr;
    unsigned int *u32 = nullptr;
    float *gdev = nullptr;
    GV_CHECK_HIP(hipMalloc(&wf, biggest * 4));
    GV_CHECK_HIP(hipMalloc(&pack, biggest));
    GV_CHECK_HIP(hipMalloc(&u32, 256));
    GV_CHECK_HIP(hipMalloc(&gdev, 256));
    auto tseed = [&](int kind, int layer, int expert) {   // the oracle's tensor seeds (oracle_layers.cpp)
        const uint64_t i = (static_cast<uint64_t>(kind) << 48) | (static_cast<uint64_t>(layer) << 24) |
                           static_cast<uint64_t>(expert);
        uint64_t x = seed * 0xD1342543DE82EF95ull + i + 0x9E3779B97F4A7C15ull;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        return x ^ (x >> 31);
    };
    int rc = 0;
    // a fresh N(0, sigma) matrix packed into the device layout; its global read back
    auto make_q4 = [&](uint64_t s, int64_t rows, int64_t cols, uint8_t *codes, uint8_t *scales, float *glob_host,
                       float *glob_dev) -> int {
        if (fill_normal(s, rows * cols, sigma, wf, st) != 0) return -1;
        if (q4_pack(wf, rows, cols, u32, pack, glob_dev ? glob_dev : gdev, st) != 0) return -1;
        Q4 tmp;
        if (q4_from_pack(pack, rows, cols, 1.0f, codes, scales, tmp, st) != 0) return -1;
        if (glob_host) {
            GV_CHECK_HIP(hipMemcpyAsync(glob_host, glob_dev ? glob_dev : gdev, 4, hipMemcpyDeviceToHost, st));
            GV_CHECK_HIP(hipStreamSynchronize(st));
        }
        return 0;
    };
    auto make_f32 = [&](uint64_t s, int64_t n, float sg, float *dst) { return fill_normal(s, n, sg, dst, st); };
    rc |= make_q4(tseed(GV_EMBED, 0, 0), V, H, const_cast<uint8_t *>(m.embed.codes), const_cast<uint8_t *>(m.embed.scales),
                  &m.embed.global, nullptr);
    rc |= make_q4(tseed(GV_LM_HEAD, 0, 0), V, H, const_cast<uint8_t *>(m.lm_head.codes),
                  const_cast<uint8_t *>(m.lm_head.scales), &m.lm_head.global, nullptr);
    rc |= make_f32(tseed(GV_FINAL_NORM, 0, 0), H, 0.02f, m.final_norm);
    if (m.has_mtp) {   // the MTP layer's fc and norms (its decoder layer: layer n_layers below)
        rc |= make_q4(tseed(GV_MTP_FC, 0, 0), H, 2 * H, const_cast<uint8_t *>(m.mtp_fc.codes),
                      const_cast<uint8_t *>(m.mtp_fc.scales), &m.mtp_fc.global, nullptr);
        rc |= make_f32(tseed(GV_MTP_NORM, 0, 0), H, 0.02f, m.mtp_norm);
        rc |= make_f32(tseed(GV_MTP_PRE_E, 0, 0), H, 0.02f, m.mtp_pre_e);
        rc |= make_f32(tseed(GV_MTP_PRE_H, 0, 0), H, 0.02f, m.mtp_pre_h);
    }
    for (int l = 0; l < static_cast<int>(m.layers.size()) && rc == 0; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        rc |= make_f32(tseed(GV_IN_NORM, l, 0), H, 0.02f, L.in_norm);
        rc |= make_f32(tseed(GV_POST_NORM, l, 0), H, 0.02f, L.post_norm);
        if (L.gdn) {   // the oracle's seeds and spreads (oracle_layers.cpp orc_model_fill)
            const int64_t nv = c.gdn_v_heads, gconv = gdn_conv_dim(c), gvd = nv * c.gdn_v_dim, K = c.conv_kernel;
            const int64_t parts[2] = {gconv, gvd};
            float *gh[2] = {&L.g_q, &L.g_k};
            int64_t off = 0;
            for (int i = 0; i < 2 && rc == 0; ++i) {   // in_proj_qkv | in_proj_z, then one permutation of the whole
                rc |= fill_normal(tseed(GV_GDN_QKV + i, l, 0), parts[i] * H, sigma, wf, st);
                rc |= q4_pack(wf, parts[i], H, u32, pack + off * (H / 16) * 9, gdev, st);
                GV_CHECK_HIP(hipMemcpyAsync(gh[i], gdev, 4, hipMemcpyDeviceToHost, st));
                GV_CHECK_HIP(hipStreamSynchronize(st));
                off += parts[i];
            }
            const float gq = L.g_q, gz = L.g_k;
            rc |= q4_from_pack(pack, gconv + gvd, H, 1.0f, const_cast<uint8_t *>(L.qkv.codes),
                               const_cast<uint8_t *>(L.qkv.scales), L.qkv, st);
            L.g_q = gq, L.g_k = gz;
            rc |= make_q4(tseed(GV_GDN_OUT, l, 0), H, gvd, const_cast<uint8_t *>(L.o.codes),
                          const_cast<uint8_t *>(L.o.scales), &L.o.global, nullptr);
            rc |= fill_normal(tseed(GV_GDN_A, l, 0), nv * H, router_sigma, wf, st);
            rc |= fill_normal(tseed(GV_GDN_B, l, 0), nv * H, router_sigma, wf + nv * H, st);
            hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(static_cast<unsigned>((2 * nv * H + 255) / 256)), dim3(256), 0,
                               st, wf, 2 * nv * H, L.gdn_ab);
            rc |= make_f32(tseed(GV_GDN_ALOG, l, 0), nv, 0.5f, L.A_log);
            rc |= make_f32(tseed(GV_GDN_DTB, l, 0), nv, 0.5f, L.dt_bias);
            rc |= make_f32(tseed(GV_GDN_CONV, l, 0), gconv * K, 0.3f, L.conv_w);
            {   // the gated norm's weight: 1 + N(0, 0.02)
                std::vector<float> gn(static_cast<size_t>(c.gdn_v_dim));
                rc |= make_f32(tseed(GV_GDN_NORM, l, 0), c.gdn_v_dim, 0.02f, wf);
                GV_CHECK_HIP(hipMemcpyAsync(gn.data(), wf, gn.size() * 4, hipMemcpyDeviceToHost, st));
                GV_CHECK_HIP(hipStreamSynchronize(st));
                for (float &v : gn) v += 1.0f;
                GV_CHECK_HIP(hipMemcpy(L.gnorm, gn.data(), gn.size() * 4, hipMemcpyHostToDevice));
            }
            // the states: a conversation's (N(0, 1) conv inputs, an N(0, 0.05) recurrent state), or zero at ctx 0
            std::vector<float> cs(static_cast<size_t>(gdn_c_floats(c)), 0.0f), ss(static_cast<size_t>(gdn_s_floats(c)), 0.0f);
            if (ctx > 0) {
                rc |= fill_normal(tseed(GV_GDN_CONV_ST, l, 0), static_cast<int64_t>(cs.size()), 1.0f, wf, st);
                GV_CHECK_HIP(hipMemcpyAsync(cs.data(), wf, cs.size() * 4, hipMemcpyDeviceToHost, st));
                GV_CHECK_HIP(hipStreamSynchronize(st));
                rc |= fill_normal(tseed(GV_GDN_S, l, 0), static_cast<int64_t>(ss.size()), 0.05f, wf, st);
                GV_CHECK_HIP(hipMemcpyAsync(ss.data(), wf, ss.size() * 4, hipMemcpyDeviceToHost, st));
                GV_CHECK_HIP(hipStreamSynchronize(st));
            }
            if (rc == 0) rc |= gdn_put_state(m, L, m.gdn_base, cs.data(), ss.data());
        }
        if (!L.gdn) {
        rc |= make_f32(tseed(GV_Q_NORM, l, 0), hd, 0.02f, L.q_norm);
        rc |= make_f32(tseed(GV_K_NORM, l, 0), hd, 0.02f, L.k_norm);
        // q | k | v packed one part at a time (each its own global), then one permutation of the whole
        const int64_t rq = nh * 2 * hd, rk = kv_row;
        float gq = 0, gk = 0, gv = 0;
        {
            const int64_t parts[3] = {rq, rk, rk};
            const int kinds[3] = {5, 6, 7};   // the oracle's ORC_Q, ORC_K, ORC_V seeds
            float *gh[3] = {&gq, &gk, &gv};
            int64_t off = 0;
            for (int i = 0; i < 3 && rc == 0; ++i) {
                rc |= fill_normal(tseed(kinds[i], l, 0), parts[i] * H, sigma, wf, st);
                rc |= q4_pack(wf, parts[i], H, u32, pack + off * (H / 16) * 9, gdev, st);
                GV_CHECK_HIP(hipMemcpyAsync(gh[i], gdev, 4, hipMemcpyDeviceToHost, st));
                GV_CHECK_HIP(hipStreamSynchronize(st));
                off += parts[i];
            }
            rc |= q4_from_pack(pack, qkv_rows(c), H, 1.0f, const_cast<uint8_t *>(L.qkv.codes),
                               const_cast<uint8_t *>(L.qkv.scales), L.qkv, st);
            L.g_q = gq, L.g_k = gk, L.g_v = gv;
        }
        rc |= make_q4(tseed(GV_O, l, 0), H, nh * hd, const_cast<uint8_t *>(L.o.codes), const_cast<uint8_t *>(L.o.scales),
                      &L.o.global, nullptr);
        }
        // router rows and the shared gate row in bf16
        rc |= fill_normal(tseed(GV_ROUTER, l, 0), static_cast<int64_t>(c.n_experts) * H, router_sigma, wf, st);
        rc |= fill_normal(tseed(GV_SHARED_GATE, l, 0), H, sigma, wf + static_cast<int64_t>(c.n_experts) * H, st);
        hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(static_cast<unsigned>((m.E1 * H + 255) / 256)), dim3(256), 0, st, wf,
                           static_cast<int64_t>(m.E1) * H, L.router);
        for (int e = 0; e <= c.n_experts && rc == 0; ++e) {
            float *gd = gdev + 4;   // device globals go straight to the experts' table
            if (e < c.n_experts) {
                rc |= make_q4(tseed(GV_EXPERT, l, 2 * e), 2 * F, H, L.gu_codes + e * m.gu_code_stride,
                              L.gu_scales + e * m.gu_scale_stride, nullptr, L.expert_globals + e * 3);
                GV_CHECK_HIP(hipMemcpyAsync(L.expert_globals + e * 3 + 1, L.expert_globals + e * 3, 4,
                                            hipMemcpyDeviceToDevice, st));
                rc |= make_q4(tseed(GV_EXPERT, l, 2 * e + 1), H, F, L.dn_codes + e * m.dn_code_stride,
                              L.dn_scales + e * m.dn_scale_stride, nullptr, L.expert_globals + e * 3 + 2);
            } else {   // the shared expert: gate and up packed apart (two globals), one gate_up permutation
                rc |= fill_normal(tseed(14, l, 0), F * H, sigma, wf, st);
                rc |= q4_pack(wf, F, H, u32, pack, L.expert_globals + e * 3, st);
                rc |= fill_normal(tseed(15, l, 0), F * H, sigma, wf, st);
                rc |= q4_pack(wf, F, H, u32, pack + F * (H / 16) * 9, L.expert_globals + e * 3 + 1, st);
                Q4 tmp;
                rc |= q4_from_pack(pack, 2 * F, H, 1.0f, L.gu_codes + e * m.gu_code_stride,
                                   L.gu_scales + e * m.gu_scale_stride, tmp, st);
                rc |= make_q4(tseed(16, l, 0), H, F, L.dn_codes + e * m.dn_code_stride,
                              L.dn_scales + e * m.dn_scale_stride, nullptr, L.expert_globals + e * 3 + 2);
            }
            (void)gd;
        }
        if (ctx > 0 && !L.gdn) {   // K then V of positions [0, ctx) in the reference's row layout, then the device's
            for (int kvi = 0; kvi < 2; ++kvi)
                rc |= fill_normal(tseed(GV_KV, l, kvi), static_cast<int64_t>(ctx) * kv_row, 1.0f,
                                  wf + static_cast<int64_t>(kvi) * ctx * kv_row, st);
            if (m.kv_i8)
                hipLaunchKernelGGL(kv8_from_rows_kernel, dim3(static_cast<unsigned>(2 * ctx * nkv)), dim3(256), 0, st,
                                   wf, ctx, static_cast<int>(nkv), static_cast<int>(hd), m.slots, L.kv8, L.kvs);
            else
                hipLaunchKernelGGL(kv_from_rows_kernel, dim3(static_cast<unsigned>((2 * ctx * kv_row + 255) / 256)),
                                   dim3(256), 0, st, wf, ctx, static_cast<int>(nkv), static_cast<int>(hd), m.slots, L.kv);
        }
    }
    (void)hipStreamSynchronize(st);
    (void)hipFree(wf);
    (void)hipFree(pack);
    (void)hipFree(u32);
    (void)hipFree(gdev);
    GV_CHECK_HIP(hipGetLastError());
    GV_REQUIRE(rc == 0, std::string("gv_model_randomize: ") + last_error());
    m.pos = ctx;
    m.mtp_last_n = 0;
    return 0;
}

int gv_model_set_position(gv_model *g, int pos) {
    GV_REQUIRE(g && pos >= 0 && pos + g->m.c.max_rows <= g->m.c.max_ctx, "gv_model_set_position: out of range");
    g->m.pos = pos;
    g->m.last_n = 0;
    g->m.mtp_last_n = 0;   // a draft then starts from a new MTP pass, not the previous conversation's
    return 0;
}

int gv_model_position(const gv_model *g) { return g ? g->m.pos : -1; }

int gv_verify(gv_model *g, const int32_t *tokens, int n, const int32_t *parents, float *logits) {
    GV_REQUIRE(g && tokens, "gv_verify: null pointer");
    Model &m = g->m;
    if (use_act_mode(m.c.exact) != 0) return -1;
    const auto &c = m.c;
    GV_REQUIRE(n >= 1 && n <= c.max_rows, "gv_verify: 1 <= n <= max_rows");
    GV_REQUIRE(m.pos + n <= c.max_ctx, "gv_verify: the context is full");
    // the step's parameters made and checked apart from the model's: a refused call leaves the last verify's
    // (which gv_verify_keep reads) and everything else as they were
    StepParams sp;
    std::memset(&sp, 0, sizeof sp);
    sp.pos = m.pos;
    sp.M = n;
    set_gdn_slots(m, sp);
    for (int i = 0; i < n; ++i) {
        GV_REQUIRE(tokens[i] >= 0 && tokens[i] < c.vocab, "gv_verify: token out of range");
        sp.tokens[i] = tokens[i];
        if (parents) {
            GV_REQUIRE(i == 0 ? parents[0] == -1 : (parents[i] >= 0 && parents[i] < i),
                       "gv_verify: parents[0] must be -1 and parents[i] < i");
            sp.depth[i] = i == 0 ? 0 : sp.depth[parents[i]] + 1;
            sp.vis[i] = (i == 0 ? 0u : sp.vis[parents[i]]) | (1u << i);
        } else {
            sp.depth[i] = i;
            sp.vis[i] = (i == 31) ? 0xFFFFFFFFu : ((1u << (i + 1)) - 1u);
        }
    }
    m.host_sp = sp;
    hipStream_t st = stream();
    GV_CHECK_HIP(hipMemcpyAsync(m.sp, &m.host_sp, sizeof sp, hipMemcpyHostToDevice, st));
    if (run_step(m, n, st) != 0) return -1;
    if (logits) {
        GV_CHECK_HIP(hipMemcpyAsync(logits, m.logits, static_cast<size_t>(n) * c.vocab * 4, hipMemcpyDeviceToHost, st));
        if (check_wait_flag(m, st) != 0) return -1;
    }
    m.last_pos = m.pos;
    m.last_n = n;
    m.pos += n;
    m.gdn_base = sp.gdn_wset + n - 1;   // (a chain's states as after its last row)
    m.hid_n = m.has_mtp ? n : 0;        // the final-normed rows the MTP layer drafts from
    m.keep_rows.clear();
    return 0;
}

int gv_verify_keep(gv_model *g, int kept, const int32_t *path) {
    GV_REQUIRE(g, "gv_verify_keep: null model");
    Model &m = g->m;
    GV_REQUIRE(m.last_n > 0 && m.pos == m.last_pos + m.last_n, "gv_verify_keep: no verify to keep from");
    GV_REQUIRE(kept >= 1 && kept <= m.last_n, "gv_verify_keep: 1 <= kept <= n");
    if (path) {
        GV_REQUIRE(path[0] == 0, "gv_verify_keep: the path starts at the root (row 0)");
        // an ancestor chain of the last verify's tree: path[j] at depth j, its parent path[j - 1] (each kept key was
        // rotated at pos + depth, so any other path would leave keys at the wrong rotary positions)
        const StepParams &sp = m.host_sp;
        for (int j = 1; j < kept; ++j) {
            GV_REQUIRE(path[j] > path[j - 1] && path[j] < m.last_n, "gv_verify_keep: path must ascend within the rows");
            GV_REQUIRE(sp.depth[path[j]] == j && ((sp.vis[path[j]] >> path[j - 1]) & 1u) != 0,
                       "gv_verify_keep: path[j] must be a depth-j child of path[j - 1] in the last verify's tree");
        }
        int *dpath = reinterpret_cast<int *>(m.rlogits);   // scratch: free between verifies
        GV_CHECK_HIP(hipMemcpyAsync(dpath, path, static_cast<size_t>(kept) * 4, hipMemcpyHostToDevice, stream()));
        const int64_t n = static_cast<int64_t>(m.c.n_layers) * m.c.n_kv_heads * m.c.head_dim;
        auto *base = reinterpret_cast<uint8_t *>(m.kv_all);
        if (m.kv_i8)
            hipLaunchKernelGGL(kv_compact_kernel<int8_t>, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                               stream(), base, m.kv_layer_bytes, m.c.n_layers, m.c.n_kv_heads, m.c.head_dim, m.slots,
                               m.last_pos, kept, dpath);
        else
            hipLaunchKernelGGL(kv_compact_kernel<_Float16>, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                               stream(), base, m.kv_layer_bytes, m.c.n_layers, m.c.n_kv_heads, m.c.head_dim, m.slots,
                               m.last_pos, kept, dpath);
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipStreamSynchronize(stream()));
    }
    m.pos = m.last_pos + kept;
    m.gdn_base = m.host_sp.gdn_wset + (path ? path[kept - 1] : kept - 1);   // the states as after the last kept row
    m.last_n = 0;
    m.keep_rows.clear();
    if (path) m.keep_rows.assign(path, path + kept);   // (the MTP layer's hidden rows: the path's)
    return 0;
}

const float *gv_model_logits(const gv_model *g) { return g ? g->m.logits : nullptr; }

int gv_model_time_kernel(gv_model *g, int cls) {
    GV_REQUIRE(g && cls < GV_K_COUNT, "gv_model_time_kernel: bad class");
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    g->m.timed_class = cls;
    g->m.events_used = 0;
    return 0;
}

int gv_model_replay(gv_model *g, int cls, int layer, int reps, float *ms_per_launch) {
    GV_REQUIRE(g && ms_per_launch && cls >= 0 && cls < GV_K_COUNT && cls != GV_K_QUANT && reps >= 1,
               "gv_model_replay: bad arguments");
    Model &m = g->m;
    if (use_act_mode(m.c.exact) != 0) return -1;
    GV_REQUIRE(layer >= 0 && layer < m.c.n_layers, "gv_model_replay: no such layer");
    GV_REQUIRE(m.last_n > 0, "gv_model_replay: no verify yet");
    const hipStream_t st = stream();
    const int saved = m.timed_class;
    m.timed_class = -1;
    // the step's row count and position as the last verify left them
    m.host_sp.pos = m.last_pos;
    GV_CHECK_HIP(hipMemcpyAsync(m.sp, &m.host_sp, sizeof(StepParams), hipMemcpyHostToDevice, st));
    // the layers the class launches on (a Gated DeltaNet class: those layers; an attention class: the others),
    // from `layer` on, cycled
    std::vector<int> on;
    const bool gdn_cls = cls >= GV_K_GDN_AB && cls <= GV_K_GDN_NORM;
    const bool attn_cls = cls == GV_K_ROPE || cls == GV_K_ATTN || cls == GV_K_MERGE;
    for (int i = 0; i < m.c.n_layers; ++i) {
        const int l = (layer + i) % m.c.n_layers;
        const bool gdn = m.layers[static_cast<size_t>(l)].gdn;
        if (!(gdn_cls && !gdn) && !(attn_cls && gdn)) on.push_back(l);
    }
    GV_REQUIRE(!on.empty(), "gv_model_replay: no layer has this kernel class");
    m.replaying = true;
    struct Done {   // (however this ends)
        Model &m;
        ~Done() { m.replaying = false; }
    } done{m};
    if (launch_class(m, cls, on[0], m.last_n, st) != 0) return -1;   // warm
    hipEvent_t e0, e1;
    GV_CHECK_HIP(hipEventCreate(&e0));
    GV_CHECK_HIP(hipEventCreate(&e1));
    GV_CHECK_HIP(hipEventRecord(e0, st));
    int rc = 0;   // launch i on the i-th such layer (cycled): each launch reads other weights than the last
    for (int i = 0; i < reps && rc == 0; ++i) rc = launch_class(m, cls, on[static_cast<size_t>(i) % on.size()], m.last_n, st);
    GV_CHECK_HIP(hipEventRecord(e1, st));
    GV_CHECK_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    GV_CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    m.timed_class = saved;
    if (rc != 0 || check_wait_flag(m, st) != 0) return -1;
    *ms_per_launch = ms / reps;
    return 0;
}

}  // extern "C"

namespace gv {
// The MoE block of layer `layer` on the M rows staged in pf.h (and the routed logits in pf.logits when given):
// the verify step's kernels for M <= max_rows (the router without a norm, the combine into a zeroed x), the
// prefill path beyond; the output in pf.out (M > max_rows) or m.x.
int moe_block(Model &m, int layer, int M, bool given, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden, E = c.n_experts;
    if (M > c.max_rows) return moe_prefill(m, layer, M, st);
    Prefill &pf = m.pf;
    m.moe_only = true;
    m.router_shared_only = given;
    m.block_h = pf.h;   // (the router reads the rows where they are; the combine writes the block's output to x)
    // at most kMaxRowsMixOut rows: the experts' up launch routes them from the logits (moe_up_kernel's route: the
    // route launch's ids, weights and slots), no route launch
    m.block_up_routes = M <= kMaxRowsMixOut;
    const bool up_route = up_routes(m, false);
    // the shared expert's gate logit and the operands: with the routed logits given and routed by the up launch,
    // prefill.hip's gate and operand roles (the router launch's values), the gate logit into the given rows' column
    // E so that the up launch routes from those rows (no copy); else the router launch, then the given logits copied
    // into its rows
    const bool lean = given && up_route && m.fused && H <= kPrefillFrontMaxH;
    int rc;
    if (lean)
        rc = prefill_gate_ops(m.layers[static_cast<size_t>(layer)].router + static_cast<int64_t>(E) * H, H, pf.h, M, E,
                              pf.logits, pf.gate, m.act_h, act_halves(H), st);
    else
        rc = launch_class(m, GV_K_ROUTER, layer, M, st);
    m.block_h = nullptr;
    m.router_shared_only = false;
    if (rc == 0 && given && !lean)                         // the routed logits as given
        rc = hipMemcpy2DAsync(m.rlogits, static_cast<size_t>(m.E1) * 4, pf.logits, static_cast<size_t>(m.E1) * 4,
                              static_cast<size_t>(E) * 4, M, hipMemcpyDeviceToDevice, st) == hipSuccess ? 0 : -1;
    m.block_logits = lean ? pf.logits : nullptr;
    for (int cls : {GV_K_ROUTE, GV_K_MOE_UP, GV_K_SWIGLU, GV_K_MOE_DOWN})
        if (rc == 0 && !(cls == GV_K_ROUTE && up_route)) rc = launch_class(m, cls, layer, M, st);
    m.block_logits = nullptr;
    m.block_up_routes = false;
    if (rc == 0) rc = launch_class(m, GV_K_COMBINE, layer, M, st);   // the block's output, no residual
    m.moe_only = false;
    return rc;
}
}  // namespace gv

extern "C" {

int gv_model_moe(gv_model *g, int layer, const float *h, int M, const float *router_logits, float *out,
                 int32_t *ids, float *weights) {
    GV_REQUIRE(g && h && out, "gv_model_moe: null pointer");
    Model &m = g->m;
    if (use_act_mode(m.c.exact) != 0) return -1;
    const auto &c = m.c;
    GV_REQUIRE(layer >= 0 && layer < c.n_layers, "gv_model_moe: no such layer");
    GV_REQUIRE(M >= 1 && M <= 16384, "gv_model_moe: 1 <= M <= 16384");
    GV_REQUIRE(M <= c.max_rows || router_logits, "gv_model_moe: more rows than max_rows need the routed logits");
    const int H = c.hidden, E = c.n_experts, K = c.top_k;
    const hipStream_t st = stream();
    if (prefill_alloc(m, M) != 0) return -1;
    Prefill &pf = m.pf;
    m.last_n = 0;   // (the last verify's parameters are replaced below: nothing is left to keep, failed or not)
    StepParams &sp = m.host_sp;
    std::memset(&sp, 0, sizeof sp);
    sp.pos = m.pos;
    sp.M = std::min(M, c.max_rows);
    GV_CHECK_HIP(hipMemcpyAsync(m.sp, &sp, sizeof sp, hipMemcpyHostToDevice, st));
    GV_CHECK_HIP(hipMemcpyAsync(pf.h, h, static_cast<size_t>(M) * H * 4, hipMemcpyHostToDevice, st));
    if (router_logits)
        GV_CHECK_HIP(hipMemcpy2DAsync(pf.logits, static_cast<size_t>(m.E1) * 4, router_logits,
                                      static_cast<size_t>(E) * 4, static_cast<size_t>(E) * 4, M,
                                      hipMemcpyHostToDevice, st));
    GV_REQUIRE(moe_block(m, layer, M, router_logits != nullptr, st) == 0,
               std::string("gv_model_moe: ") + last_error());
    pf.M = M;
    pf.given = router_logits != nullptr;
    pf.layer = layer;
    const bool big = M > c.max_rows;
    GV_CHECK_HIP(hipMemcpyAsync(out, big ? pf.out : m.x, static_cast<size_t>(M) * H * 4, hipMemcpyDeviceToHost, st));
    if (ids)
        GV_CHECK_HIP(hipMemcpyAsync(ids, big ? pf.ids : m.route_ids + static_cast<int64_t>(layer) * c.max_rows * K,
                                    static_cast<size_t>(M) * K * 4, hipMemcpyDeviceToHost, st));
    if (weights)
        GV_CHECK_HIP(hipMemcpyAsync(weights, big ? pf.w : m.route[layer].weight, static_cast<size_t>(M) * K * 4,
                                    hipMemcpyDeviceToHost, st));
    if (check_wait_flag(m, st) != 0) return -1;   // (synchronizes the stream)
    m.last_n = 0;   // the step's state is this block's, not a verify's
    return 0;
}

int gv_model_layer(gv_model *g, int layer, const float *x_in, int n, const int32_t *parents, float *x_mid,
                   float *x_out, int32_t *ids) {
    GV_REQUIRE(g && x_in, "gv_model_layer: null pointer");
    Model &m = g->m;
    if (use_act_mode(m.c.exact) != 0) return -1;
    const auto &c = m.c;
    GV_REQUIRE(layer >= 0 && layer < c.n_layers, "gv_model_layer: no such layer");
    GV_REQUIRE(n >= 1 && n <= c.max_rows && m.pos + n <= c.max_ctx, "gv_model_layer: 1 <= n <= max_rows, in context");
    m.last_n = 0;   // (the last verify's parameters are replaced below: nothing is left to keep, failed or not)
    StepParams &sp = m.host_sp;
    std::memset(&sp, 0, sizeof sp);
    sp.pos = m.pos;
    sp.M = n;
    set_gdn_slots(m, sp);   // (the rows' states go to the other set: the base stays)
    for (int i = 0; i < n; ++i) {
        if (parents) {
            GV_REQUIRE(i == 0 ? parents[0] == -1 : (parents[i] >= 0 && parents[i] < i), "gv_model_layer: parents");
            sp.depth[i] = i == 0 ? 0 : sp.depth[parents[i]] + 1;
            sp.vis[i] = (i == 0 ? 0u : sp.vis[parents[i]]) | (1u << i);
        } else {
            sp.depth[i] = i;
            sp.vis[i] = (i == 31) ? 0xFFFFFFFFu : ((1u << (i + 1)) - 1u);
        }
    }
    const hipStream_t st = stream();
    const int H = c.hidden;
    GV_CHECK_HIP(hipMemcpyAsync(m.sp, &sp, sizeof sp, hipMemcpyHostToDevice, st));
    GV_CHECK_HIP(hipMemcpyAsync(m.x, x_in, static_cast<size_t>(n) * H * 4, hipMemcpyHostToDevice, st));
    // the layer's input norm and operands (in a step: the previous layer's combine, or the embedding)
    LayerW &L = m.layers[static_cast<size_t>(layer)];
    if (quantize_act(m.x, H, n, H, L.in_norm, c.eps, m.act_h, act_halves(H), nullptr, 0, st) != 0) return -1;
    for (int cls : {GV_K_QKV, GV_K_GDN_AB, GV_K_GDN_CONV, GV_K_GDN_CORE, GV_K_GDN_NORM, GV_K_ROPE, GV_K_ATTN, GV_K_MERGE,
                    GV_K_O})
        if (launch_class(m, cls, layer, n, st) != 0) return -1;
    if (x_mid) GV_CHECK_HIP(hipMemcpyAsync(x_mid, m.x, static_cast<size_t>(n) * H * 4, hipMemcpyDeviceToHost, st));
    for (int cls : {GV_K_ROUTER, GV_K_ROUTE, GV_K_MOE_UP, GV_K_SWIGLU, GV_K_MOE_DOWN, GV_K_COMBINE})
        if (launch_class(m, cls, layer, n, st) != 0) return -1;
    if (x_out) GV_CHECK_HIP(hipMemcpyAsync(x_out, m.x, static_cast<size_t>(n) * H * 4, hipMemcpyDeviceToHost, st));
    if (ids)
        GV_CHECK_HIP(hipMemcpyAsync(ids, m.route_ids + static_cast<int64_t>(layer) * c.max_rows * c.top_k,
                                    static_cast<size_t>(n) * c.top_k * 4, hipMemcpyDeviceToHost, st));
    if (check_wait_flag(m, st) != 0) return -1;
    m.last_n = 0;   // nothing to keep: the position is unchanged
    return 0;
}

int gv_model_gdn_state(const gv_model *g, int layer, float *conv, float *S) {
    GV_REQUIRE(g && layer >= 0 && layer < g->m.c.n_layers, "gv_model_gdn_state: no such layer");
    const Model &m = g->m;
    const LayerW &L = m.layers[static_cast<size_t>(layer)];
    GV_REQUIRE(L.gdn, "gv_model_gdn_state: not a Gated DeltaNet layer");
    return gdn_get_state(m, L, m.gdn_base, conv, S);
}

int gv_model_moe_replay(gv_model *g, int reps, float *ms_per_block) {
    GV_REQUIRE(g && ms_per_block && reps >= 1, "gv_model_moe_replay: bad arguments");
    Model &m = g->m;
    if (use_act_mode(m.c.exact) != 0) return -1;
    GV_REQUIRE(m.pf.M > 0, "gv_model_moe_replay: no gv_model_moe call to replay");
    const hipStream_t st = stream();
    if (moe_block(m, m.pf.layer, m.pf.M, m.pf.given, st) != 0) return -1;   // warm
    hipEvent_t e0, e1;
    GV_CHECK_HIP(hipEventCreate(&e0));
    GV_CHECK_HIP(hipEventCreate(&e1));
    GV_CHECK_HIP(hipEventRecord(e0, st));
    int rc = 0;
    for (int i = 0; i < reps && rc == 0; ++i)   // launch i on layer (layer + i) mod n_layers: other weights each time
        rc = moe_block(m, (m.pf.layer + i) % m.c.n_layers, m.pf.M, m.pf.given, st);
    GV_CHECK_HIP(hipEventRecord(e1, st));
    GV_CHECK_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    GV_CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != 0 || check_wait_flag(m, st) != 0) return -1;
    *ms_per_block = ms / reps;
    return 0;
}

int gv_model_trace(gv_model *g, int on) {
    GV_REQUIRE(g, "gv_model_trace: null model");
    Model &m = g->m;
    const size_t bytes = static_cast<size_t>(GV_K_COUNT) * kTraceWgs * 8 * 8;
    if (on && !m.trace) {
        GV_CHECK_HIP(hipMalloc(&m.trace, bytes));
        GV_CHECK_HIP(hipMemset(m.trace, 0, bytes));
    }
    uint64_t *p = on ? m.trace : nullptr;
    // no kernel of the library's stream may run while the pointer changes: the stream is non-blocking, so the
    // symbol copies below would not wait for it, and a kernel reading the pointer mid-copy may see half of each
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    GV_CHECK_HIP(hipDeviceSynchronize());
    GV_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &p, sizeof p));
    const int rc = trace_set_q4(p) != 0 ? -1 : trace_set_gdn(p);
    GV_CHECK_HIP(hipDeviceSynchronize());
    return rc;
}

int64_t gv_model_trace_read(gv_model *g, uint64_t *out, int64_t n) {
    GV_REQUIRE(g && out && n >= 0 && g->m.trace, "gv_model_trace_read: no trace");
    const int64_t have = static_cast<int64_t>(GV_K_COUNT) * kTraceWgs * 8;
    const int64_t k = std::min(n, have);
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    GV_CHECK_HIP(hipMemcpy(out, g->m.trace, static_cast<size_t>(k) * 8, hipMemcpyDeviceToHost));
    return k;
}

int gv_model_set_graphs(gv_model *g, int on) {
    GV_REQUIRE(g, "gv_model_set_graphs: null model");
    g->m.use_graphs = on != 0;
    return 0;
}

int gv_model_set_fused(gv_model *g, int on) {
    GV_REQUIRE(g, "gv_model_set_fused: null model");
    Model &m = g->m;
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    GV_REQUIRE(on >= 0 && on <= 2, "gv_model_set_fused: 0, 1 or 2");
    m.fused = on != 0;
    m.route_in_up = on == 1;
    for (auto &ge : m.graphs)   // the graphs hold the other launches: captured again on the next steps
        if (ge) {
            (void)hipGraphExecDestroy(ge);
            ge = nullptr;
        }
    for (bool &s : m.seen) s = false;
    return 0;
}

int gv_model_kernel_time(gv_model *g, float *total_ms, int *launches) {
    GV_REQUIRE(g && total_ms && launches, "gv_model_kernel_time: null pointer");
    Model &m = g->m;
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    float sum = 0.0f;
    for (size_t i = 0; i + 1 < m.events_used; i += 2) {
        float ms = 0.0f;
        GV_CHECK_HIP(hipEventElapsedTime(&ms, m.events[i], m.events[i + 1]));
        sum += ms;
    }
    *total_ms = sum;
    *launches = static_cast<int>(m.events_used / 2);
    return 0;
}

int gv_model_route_ids(const gv_model *g, int32_t *out) {
    GV_REQUIRE(g && out && g->m.last_n > 0, "gv_model_route_ids: no verify yet");
    const auto &c = g->m.c;
    const int n = g->m.last_n;
    for (int l = 0; l < c.n_layers; ++l)
        GV_CHECK_HIP(hipMemcpy(out + static_cast<size_t>(l) * n * c.top_k,
                               g->m.route_ids + static_cast<size_t>(l) * c.max_rows * c.top_k,
                               static_cast<size_t>(n) * c.top_k * 4, hipMemcpyDeviceToHost));
    return 0;
}

}  // extern "C"
