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

#include "mfma_gemv.hpp"
#include "model.hpp"

namespace gv {

hipStream_t stream();
int ensure_init();

// ---------------------------------------------------------------- kernels
// the rows' embeddings: dequant_row of the embedding matrix (pack.cpp:356-366), bit for bit
__global__ void embed_kernel(Q4 w, const StepParams *__restrict__ sp, float *__restrict__ x) {
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const int64_t r = sp->tokens[t];
    for (int64_t wi = threadIdx.x; wi < w.cols / 8; wi += blockDim.x) {   // the row's code words (tile layout)
        uint32_t word, sb;
        tq4_word(w, r, wi, word, sb);
        const float s = __fmul_rn(e4m3_to_f32(sb), w.global);
        float *o = x + static_cast<int64_t>(t) * w.cols + wi * 8;
        for (int b = 0; b < 8; ++b)
            o[b] = __fmul_rn(static_cast<float>(2 * static_cast<int>((word >> (4 * b)) & 15u) - 15), s);
    }
}

__device__ inline double block_sum_double(double v, double *red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int o = blockDim.x / 2; o > 0; o >>= 1) {
        if (static_cast<int>(threadIdx.x) < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

// The device KV cache of one layer: K [nkv][slots][hd] and V [nkv][slots / 64][hd][64] in fp16 (V transposed in
// blocks of kAttnBlock positions, so that the MFMA operands of both products are contiguous loads).
__device__ __host__ inline int64_t k_index(int64_t slots, int hd, int kh, int64_t slot, int d) {
    return (static_cast<int64_t>(kh) * slots + slot) * hd + d;
}
__device__ __host__ inline int64_t v_index(int64_t slots, int hd, int nkv, int kh, int64_t slot, int d) {
    return static_cast<int64_t>(nkv) * slots * hd +
           ((static_cast<int64_t>(kh) * (slots / kAttnBlock) + slot / kAttnBlock) * hd + d) * kAttnBlock + slot % kAttnBlock;
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
                                                      _Float16 *__restrict__ kv, int64_t slots) {
    const int t = blockIdx.x, head = blockIdx.y, i = threadIdx.x;
    if (t >= sp->M) return;
    __shared__ double red[256];
    __shared__ float v[256];
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
    const float xv = i < hd ? src[i] : 0.0f;
    if (kind == 2) {
        if (i < hd) kv[v_index(slots, hd, nkv, kh, slot, i)] = static_cast<_Float16>(xv);
        return;
    }
    const double ss = block_sum_double(static_cast<double>(xv) * static_cast<double>(xv), red);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(ss / static_cast<double>(hd)), eps)));
    if (i < hd) v[i] = __fmul_rn(__fmul_rn(xv, inv), __fadd_rn(1.0f, nw[i]));
    __syncthreads();
    if (i >= hd) return;
    const int p = sp->pos + sp->depth[t];
    float out = v[i];
    if (i < half) {
        const float c = cos_t[static_cast<int64_t>(p) * half + i], s = sin_t[static_cast<int64_t>(p) * half + i];
        out = __fsub_rn(__fmul_rn(v[i], c), __fmul_rn(v[i + half], s));
    } else if (i < 2 * half) {
        const int j = i - half;
        const float c = cos_t[static_cast<int64_t>(p) * half + j], s = sin_t[static_cast<int64_t>(p) * half + j];
        out = __fadd_rn(__fmul_rn(v[i], c), __fmul_rn(v[j], s));
    }
    if (kind == 0) {   // the query as two halves, hi + lo, for near-fp32 scores from fp16 products
        const int64_t qo = (static_cast<int64_t>(t) * nh + head) * hd + i;
        const _Float16 hi = static_cast<_Float16>(out);
        q_out[qo] = hi;
        q_out[qo + static_cast<int64_t>(sp->M) * nh * hd] = static_cast<_Float16>(out - static_cast<float>(hi));
    } else {
        kv[k_index(slots, hd, kh, slot, i)] = static_cast<_Float16>(out);
    }
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Split-KV attention on the matrix cores: a wave per (16 queries, block of 64 positions, KV head); the queries of a
// KV head are its query heads x the rows. S^T = K Q^T (v_mfma_f32_16x16x32_f16: fp16 keys, the queries as hi + lo
// fp16 halves, fp32 sums), masked to the context plus each row's visible rows, then per query the block's
// maximum, the weights exp(s - max) and their sum; O^T = V^T P^T with the weights as hi + lo halves. Writes the block's
// partial (weighted values, max, sum) as attend_heads does per block (model.cpp:3894-4018); attn_merge joins them.
__global__ __launch_bounds__(64) void attn_mfma_kernel(const _Float16 *__restrict__ q16, const _Float16 *__restrict__ kv,
                                                       int64_t slots, int nh, int nkv, int hd,
                                                       const StepParams *__restrict__ sp, float *__restrict__ parts,
                                                       int nb_max) {
    const int qt = blockIdx.x, b = blockIdx.y, kh = blockIdx.z;
    const int pos = sp->pos, M = sp->M, total = pos + M;
    const int group = nh / nkv, NQ = group * M;
    const int s0 = b * kAttnBlock;
    if (s0 >= total || qt * 16 >= NQ) return;
    const int l = threadIdx.x, lq = l % 16, lg = l / 16;
    const int qi = qt * 16 + lq;
    const bool qvalid = qi < NQ;
    const int tq = qvalid ? qi / group : 0, hq = kh * group + (qvalid ? qi % group : 0);
    const int nch = hd / 32;
    // the queries as B operands (hi and lo halves): dims ch * 32 + 8 lg .. + 8 of query lq
    half8 qb[8], ql[8];
    const int64_t qlo = static_cast<int64_t>(M) * nh * hd;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
        const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
        const int64_t qo = (static_cast<int64_t>(tq) * nh + hq) * hd + ch * 32 + 8 * lg;
        qb[ch] = (qvalid && ch < nch) ? *reinterpret_cast<const half8 *>(q16 + qo) : z;
        ql[ch] = (qvalid && ch < nch) ? *reinterpret_cast<const half8 *>(q16 + qlo + qo) : z;
    }
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(hd)));
    const uint32_t vis = qvalid ? sp->vis[tq] : 0u;
    float sc[4][4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
        float4v c = {0, 0, 0, 0};
        const _Float16 *krow = kv + k_index(slots, hd, kh, s0 + pt * 16 + lq, 8 * lg);
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
            if (ch >= nch) break;
            const half8 a = *reinterpret_cast<const half8 *>(krow + ch * 32);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[ch], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[ch], c, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {   // S^T[position pt*16 + 4 lg + r][query lq]
            const int slot = s0 + pt * 16 + 4 * lg + r;
            const bool ok = qvalid && slot < total && (slot < pos || ((vis >> (slot - pos)) & 1u));
            sc[pt][r] = ok ? c[r] * scale : -__builtin_inff();
            mx = fmaxf(mx, sc[pt][r]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float lsum = 0.0f;
    half4 pe[4], pl[4];   // the weights as hi + lo halves
#pragma unroll
    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = sc[pt][r] == -__builtin_inff() ? 0.0f : expf(sc[pt][r] - mx);
            const _Float16 eh = static_cast<_Float16>(e);
            pe[pt][r] = eh;
            pl[pt][r] = static_cast<_Float16>(e - static_cast<float>(eh));
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
    const _Float16 *vblk = kv + v_index(slots, hd, nkv, kh, s0, 0);   // [hd][64] of this block
    for (int dt = 0; dt < hd / 16; ++dt) {
        float4v c = {0, 0, 0, 0};
        const _Float16 *vrow = vblk + static_cast<int64_t>(dt * 16 + lq) * kAttnBlock;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const half4 lo = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 4 * lg);
            const half4 hi = *reinterpret_cast<const half4 *>(vrow + kc * 32 + 16 + 4 * lg);
            const half8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[kc], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pbl[kc], c, 0, 0, 0);
        }
        // O^T[dim dt*16 + 4 lg + r][query lq]
        if (qvalid) *reinterpret_cast<float4 *>(dst + dt * 16 + 4 * lg) = make_float4(c[0], c[1], c[2], c[3]);
    }
    if (qvalid && lg == 0) {
        dst[hd] = mx;
        dst[hd + 1] = lsum;
    }
}

// The blocks joined per (row, head): exp(block max - max), the sums, 1 / sum, times sigmoid(gate)
// (model.cpp:3830-3855). A workgroup per (row, head); the blocks' weights computed once.
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ parts, const float *__restrict__ qkv,
                                                         int64_t ldq, int nh, int hd, int nb_max,
                                                         const StepParams *__restrict__ sp, float *__restrict__ core) {
    __shared__ float fw[1024];
    __shared__ float lsum;
    const int t = blockIdx.x, h = blockIdx.y;
    if (t >= sp->M) return;
    const int nbw = (sp->pos + sp->M + kAttnBlock - 1) / kAttnBlock;
    const float *base = parts + ((static_cast<int64_t>(t) * nh + h) * nb_max) * (hd + 2);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (wave == 0) {
        float mx = -__builtin_inff();
        for (int b = lane; b < nbw; b += 64) mx = fmaxf(mx, base[b * (hd + 2) + hd]);
        mx = wave_max(mx);
        float l = 0.0f;
        for (int b = lane; b < nbw; b += 64) {
            const float mb = base[b * (hd + 2) + hd];
            const float f = mb == -__builtin_inff() ? 0.0f : expf(__fsub_rn(mb, mx));
            fw[b] = f;
            l = __builtin_fmaf(base[b * (hd + 2) + hd + 1], f, l);
        }
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
        if (lane == 0) lsum = l;
    }
    __syncthreads();
    const float inv = __fdiv_rn(1.0f, lsum);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (int b = 0; b < nbw; ++b) o = __builtin_fmaf(base[b * (hd + 2) + d], fw[b], o);
        const float gate = qkv[t * ldq + static_cast<int64_t>(h) * 2 * hd + hd + d];
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gate)));
        core[(static_cast<int64_t>(t) * nh + h) * hd + d] = __fmul_rn(__fmul_rn(o, inv), sig);
    }
}

// Router logits: bf16 rows [E + 1][H] (the shared expert's gate row last) times the post-norm rows, eight partial
// sums per row in the reference's fixed order (bf16_row_dots, kernels.cpp:1446-1483). A wave per row, its lanes
// 8 tokens x 8 partial sums; loads in chunks of 32 columns ahead of the sequential sums.
__global__ __launch_bounds__(256) void router_kernel(const uint16_t *__restrict__ w, int E1, int H,
                                                     const float *__restrict__ h, const StepParams *__restrict__ sp,
                                                     float *__restrict__ logits) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x * 4 + wave;
    if (r >= E1) return;
    const int M = sp->M;
    const uint16_t *row = w + static_cast<int64_t>(r) * H;
    for (int t0 = 0; t0 < M; t0 += 8) {
        const int t = t0 + lane / 8, j = lane % 8;
        const bool live = t < M;
        const float *x = h + static_cast<int64_t>(live ? t : 0) * H;
        float acc = 0.0f;
        for (int c0 = 0; c0 < H; c0 += 256) {
            float wf[32], xv[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                wf[u] = __uint_as_float(static_cast<uint32_t>(row[c0 + u * 8 + j]) << 16);
                xv[u] = x[c0 + u * 8 + j];
            }
#pragma unroll
            for (int u = 0; u < 32; ++u) acc = __fadd_rn(acc, __fmul_rn(wf[u], xv[u]));
        }
        const float s = __fadd_rn(acc, __shfl_down(acc, 4, 64));          // lanes j < 4: a_j + a_{j+4}
        const float s2 = __fadd_rn(s, __shfl_down(s, 1, 64));             // j = 0: s0 + s1, j = 2: s2 + s3
        const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));           // j = 0: (s0 + s1) + (s2 + s3)
        if (j == 0 && live) logits[static_cast<int64_t>(t) * E1 + r] = s3;
    }
}

// The route (route_topk, model.cpp:4021-4065): softmax over the experts (max, expf, the sum in index order, divide),
// the top K by probability with ties to the lower index, the weights p / (their sum in rank order); the shared
// expert's gate sigmoid(logit); then the slots (distinct experts ascending, the shared one last) and their picks
// ordered by (expert, token, rank), each pick placed by counting, so the order never depends on timing.
__global__ __launch_bounds__(1024) void route_kernel(const float *__restrict__ logits, int E, int K,
                                                    const StepParams *__restrict__ sp, RouteState *__restrict__ rs,
                                                    int32_t *__restrict__ ids_out) {
    __shared__ float p[kMaxRows][256];
    __shared__ int ids[kMaxRows * 16];
    __shared__ int cnt[257], start[257], slot_of[257];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int M = sp->M, E1 = E + 1;
    for (int e = threadIdx.x; e <= E; e += blockDim.x) cnt[e] = 0;
    for (int t = wave; t < M; t += waves) {
        const float *lg = logits + static_cast<int64_t>(t) * E1;
        float v[4];
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            v[i] = e < E ? lg[e] : -__builtin_inff();
            mx = fmaxf(mx, v[i]);
        }
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            if (e < E) p[t][e] = expf(__fsub_rn(v[i], mx));
        }
        __builtin_amdgcn_wave_barrier();
        float sum = 0.0f;
        if (lane == 0) {   // index order, as the reference; four values a load
            int e = 0;
            for (; e + 4 <= E; e += 4) {
                const float4 v4 = *reinterpret_cast<const float4 *>(&p[t][e]);
                sum = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(sum, v4.x), v4.y), v4.z), v4.w);
            }
            for (; e < E; ++e) sum = __fadd_rn(sum, p[t][e]);
        }
        sum = __shfl(sum, 0, 64);
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = lane + 64 * i;
            pv[i] = e < E ? __fdiv_rn(p[t][e], sum) : -1.0f;
        }
        float top = 0.0f, mine = 0.0f;
        for (int k = 0; k < K; ++k) {
            float bv = -1.0f;
            int bi = E;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = lane + 64 * i;
                if (pv[i] > bv || (pv[i] == bv && e < bi)) bv = pv[i], bi = e;
            }
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) bv = ov, bi = oi;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane + 64 * i == bi) pv[i] = -1.0f;   // taken
            if (lane == k) mine = bv;
            if (lane == 0) ids[t * 16 + k] = bi;
            top = __fadd_rn(top, bv);   // rank order
        }
        if (lane < K) {
            rs->weight[t * K + lane] = __fdiv_rn(mine, top);
            ids_out[t * K + lane] = ids[t * 16 + lane];
        }
        if (lane == 0) rs->gate[t] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-lg[E])));
    }
    __syncthreads();
    // counts per expert (the shared expert, E, once per row)
    for (int i = threadIdx.x; i < M * K; i += blockDim.x) atomicAdd(&cnt[ids[(i / K) * 16 + i % K]], 1);
    if (threadIdx.x == 0) cnt[E] = M;
    __syncthreads();
    if (threadIdx.x == 0) {   // exclusive scans over 257 counters: starts and slot numbers
        int run = 0, u = 0;
        for (int e = 0; e <= E; ++e) {
            start[e] = run;
            slot_of[e] = cnt[e] > 0 ? u : -1;
            run += cnt[e];
            u += cnt[e] > 0;
        }
        rs->n_slots = u;
        rs->n_picks = run;
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += blockDim.x)
        if (slot_of[e] >= 0) {
            rs->slot_expert[slot_of[e]] = e;
            rs->slot_start[slot_of[e]] = start[e];
            rs->slot_count[slot_of[e]] = cnt[e];
        }
    // pick (t, k) of expert e goes after the earlier rows' picks of e (a row picks an expert at most once)
    for (int i = threadIdx.x; i < M * (K + 1); i += blockDim.x) {
        const int t = i / (K + 1), k = i % (K + 1);
        const int e = k < K ? ids[t * 16 + k] : E;
        int before = 0;
        if (k < K) {
            for (int t2 = 0; t2 < t; ++t2)
                for (int k2 = 0; k2 < K; ++k2) before += ids[t2 * 16 + k2] == e;
        } else {
            before = t;
        }
        const int pk = start[e] + before;
        rs->pick_token[pk] = t;
        rs->pick_of[t * (K + 1) + k] = pk;
    }
}

// The experts' products on the matrix cores, a workgroup per (slot, row tiles): UP takes gate_up [2F x H] against
// the post-norm rows of the slot's tokens, DOWN takes down [H x F] against the slot's picks' SwiGLU rows; each
// pick's rows go to out [pick][rows].
template <int KW, int NTT, int WMAX, bool UP>
__global__ __launch_bounds__(64 * WMAX) void moe_mfma_kernel(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales,
                                                        size_t code_stride, size_t scale_stride, int64_t rows, int K,
                                                        const float *__restrict__ globals, int half_rows,
                                                        const _Float16 *__restrict__ act, int64_t act_stride,
                                                        const RouteState *__restrict__ rs, float *__restrict__ out,
                                                        int tiles_per_wg) {
    extern __shared__ f4 part_lds[];
    __shared__ uint2 tab[256];
    fill_e4m3_table(tab);
    __syncthreads();
    const int u = blockIdx.x;
    if (u >= rs->n_slots) return;
    const int e = rs->slot_expert[u], start = rs->slot_start[u], cnt = rs->slot_count[u];
    const int64_t ntiles = tiles_rows(rows);
    const int64_t t0 = static_cast<int64_t>(blockIdx.y) * tiles_per_wg;
    const int64_t t1 = t0 + tiles_per_wg < ntiles ? t0 + tiles_per_wg : ntiles;
    if (t0 >= ntiles) return;
    const float g0 = globals[e * 3], g1 = globals[e * 3 + 1], g2 = globals[e * 3 + 2];
    mfma_tiles<KW, NTT>(
        codes + static_cast<size_t>(e) * code_stride, scales + static_cast<size_t>(e) * scale_stride, rows,
        K / kSuperK, 0, t0, t1,
        cnt,
        [&](int j) {
            const int64_t src = UP ? rs->pick_token[start + j] : start + j;
            return act + src * act_stride;
        },
        [&](int64_t row, int j, float v) {
            const float gl = UP ? (row < half_rows ? g0 : g1) : g2;
            out[static_cast<int64_t>(start + j) * rows + row] = v * gl;
        },
        part_lds, tab);
}

// per pick: silu(gate) * up (kernels.hpp:141), quantized for down
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float *__restrict__ gu, int F,
                                                           const RouteState *__restrict__ rs,
                                                           _Float16 *__restrict__ act_m) {
    extern __shared__ uint4 lds_u4[];
    float *m = reinterpret_cast<float *>(lds_u4);
    const int p = blockIdx.x;
    if (p >= rs->n_picks) return;
    const float *row = gu + static_cast<int64_t>(p) * 2 * F;
    for (int i = threadIdx.x; i < F; i += blockDim.x) {
        const float x = row[i];
        m[i] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), row[F + i]);
    }
    __syncthreads();
    act16_row(m, F, act_m + static_cast<int64_t>(p) * act_halves(F), false);
}

// x += sigmoid(gate) x shared + sum_k w_k y_k in rank order (model.cpp:4554-4585, :5363-5365); a workgroup per
// (row, 256 columns)
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y, int H, int K,
                                                      const RouteState *__restrict__ rs,
                                                      const StepParams *__restrict__ sp, float *__restrict__ x) {
    const int t = blockIdx.x, i = blockIdx.y * blockDim.x + threadIdx.x;
    if (t >= sp->M || i >= H) return;
    const float gs = rs->gate[t];
    float o = __fmul_rn(gs, y[static_cast<int64_t>(rs->pick_of[t * (K + 1) + K]) * H + i]);
    for (int k = 0; k < K; ++k) {
        const float wk = rs->weight[t * K + k];
        if (wk == 0.0f) continue;
        o = __fadd_rn(o, __fmul_rn(wk, y[static_cast<int64_t>(rs->pick_of[t * (K + 1) + k]) * H + i]));
    }
    x[static_cast<int64_t>(t) * H + i] = __fadd_rn(x[static_cast<int64_t>(t) * H + i], o);
}

// verify_keep of a tree: the kept path's keys and values moved to the kept slots in every layer; a thread per
// (layer, KV head, dim)
__global__ void kv_compact_kernel(_Float16 *kv_all, int n_layers, int nkv, int hd, int64_t slots, int pos, int kept,
                                  const int *__restrict__ path) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(n_layers) * nkv * hd) return;
    const int l = static_cast<int>(i / (static_cast<int64_t>(nkv) * hd)), kh = static_cast<int>((i / hd) % nkv);
    const int d = static_cast<int>(i % hd);
    _Float16 *kv = kv_all + static_cast<int64_t>(l) * 2 * nkv * slots * hd;
    for (int j = 1; j < kept; ++j) {   // ascending: path[j] >= j, so no source is overwritten before it is read
        if (path[j] == j) continue;
        kv[k_index(slots, hd, kh, pos + j, d)] = kv[k_index(slots, hd, kh, pos + path[j], d)];
        kv[v_index(slots, hd, nkv, kh, pos + j, d)] = kv[v_index(slots, hd, nkv, kh, pos + path[j], d)];
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

template <int KW, int NTT, int WMAX, bool UP>
int launch_moe(const Model &m, const LayerW &L, int waves, hipStream_t st) {
    const int64_t H = m.c.hidden, F = m.c.moe_ff;
    const int64_t rows = UP ? 2 * F : H, cols = UP ? H : F;
    const int64_t ntiles = tiles_rows(rows);
    // ~8 workgroups a slot, the waves' partial sums within 48 KB of LDS
    const int64_t cap = waves > 1 ? std::max(1, 48 / (waves * NTT)) : 64;
    const int per = static_cast<int>(std::min<int64_t>(cap, (ntiles + 7) / 8));
    const int tiles = static_cast<int>((ntiles + per - 1) / per);
    const size_t lds = waves > 1 ? static_cast<size_t>(per) * waves * NTT * 1024 : 0;
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&moe_mfma_kernel<KW, NTT, WMAX, UP>), 64 * 1024, granted) != 0)
        return -1;
    hipLaunchKernelGGL((moe_mfma_kernel<KW, NTT, WMAX, UP>), dim3(m.max_slots, tiles), dim3(64 * waves), lds, st,
                       UP ? L.gu_codes : L.dn_codes, UP ? L.gu_scales : L.dn_scales,
                       UP ? m.gu_code_stride : m.dn_code_stride, UP ? m.gu_scale_stride : m.dn_scale_stride, rows,
                       static_cast<int>(cols), L.expert_globals, static_cast<int>(F), UP ? m.act_h : m.act_m,
                       act_halves(cols), m.route + (&L - &m.layers[0]), UP ? m.gu_out : m.y, per);
    return 0;
}

template <bool UP>
int moe_launch(const Model &m, const LayerW &L, int ntt, int kw, int waves, hipStream_t st) {
    if (ntt == 1) {
        if (kw == 16) return launch_moe<16, 1, 8, UP>(m, L, waves, st);
        if (kw == 8) return launch_moe<8, 1, 8, UP>(m, L, waves, st);
        return launch_moe<4, 1, 8, UP>(m, L, waves, st);
    }
    if (kw == 8) return launch_moe<8, 2, 8, UP>(m, L, waves, st);
    return launch_moe<4, 2, 8, UP>(m, L, waves, st);
}

int moe_products(const Model &m, const LayerW &L, int M, bool up, hipStream_t st) {
    const int ntt = M <= 16 ? 1 : 2;
    int waves, kw;
    GV_REQUIRE(mfma_split(up ? m.c.hidden : m.c.moe_ff, ntt, waves, kw), "moe: K too wide for one launch");
    return up ? moe_launch<true>(m, L, ntt, kw, waves, st) : moe_launch<false>(m, L, ntt, kw, waves, st);
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

int run_layers(Model &m, int M, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const int64_t abH = act_halves(H), abC = act_halves(static_cast<int64_t>(nh) * hd);
    {
        Tick tk(m, GV_K_EMBED, st);
        hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, st, m.embed, m.sp, m.x);
    }
    for (int l = 0; l < c.n_layers; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        {
            Tick tk(m, GV_K_QUANT, st);
            if (quantize_act(m.x, H, M, H, L.in_norm, c.eps, 0, m.act_h, abH, nullptr, 0, st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_QKV, st);
            if (gemv_q4(L.qkv, m.act_h, abH, M, qkv_out(m, L), st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_ROPE, st);
            hipLaunchKernelGGL(qk_rope_kernel, dim3(M, nh + 2 * nkv), dim3(256), 0, st, m.qkv_out, L.qkv.rows, nh, nkv, hd,
                               c.rope_dim / 2, L.q_norm, L.k_norm, c.eps, m.rope_cos, m.rope_sin, m.sp, m.q16, L.kv,
                               m.slots);
        }
        const int qtiles = (nh / nkv * M + 15) / 16;
        {
            Tick tk(m, GV_K_ATTN, st);
            hipLaunchKernelGGL(attn_mfma_kernel, dim3(qtiles, m.kv_blocks, nkv), dim3(64), 0, st, m.q16, L.kv, m.slots, nh,
                               nkv, hd, m.sp, m.parts, m.kv_blocks);
        }
        {
            Tick tk(m, GV_K_MERGE, st);
            hipLaunchKernelGGL(attn_merge_kernel, dim3(M, nh), dim3(256), 0, st, m.parts, m.qkv_out, L.qkv.rows, nh, hd,
                               m.kv_blocks, m.sp, m.core);
        }
        {
            Tick tk(m, GV_K_QUANT, st);
            if (quantize_act(m.core, nh * hd, M, nh * hd, nullptr, 0.0f, 0, m.act_core, abC, nullptr, 0, st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_O, st);
            if (gemv_q4(L.o, m.act_core, abC, M, gemv_out(m.x, H, L.o.global, 1), st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_QUANT, st);
            if (quantize_act(m.x, H, M, H, L.post_norm, c.eps, 0, m.act_h, abH, m.h, H, st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_ROUTER, st);
            hipLaunchKernelGGL(router_kernel, dim3((m.E1 + 3) / 4), dim3(256), 0, st, L.router, m.E1, H, m.h, m.sp,
                               m.rlogits);
        }
        {
            Tick tk(m, GV_K_ROUTE, st);
            hipLaunchKernelGGL(route_kernel, dim3(1), dim3(1024), 0, st, m.rlogits, c.n_experts, c.top_k, m.sp, m.route + l,
                               m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k);
        }
        {
            Tick tk(m, GV_K_MOE_UP, st);
            if (moe_products(m, L, M, true, st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_SWIGLU, st);
            hipLaunchKernelGGL(swiglu_quant_kernel, dim3(m.max_picks), dim3(256), static_cast<size_t>(c.moe_ff) * 4, st,
                               m.gu_out, c.moe_ff, m.route + l, m.act_m);
        }
        {
            Tick tk(m, GV_K_MOE_DOWN, st);
            if (moe_products(m, L, M, false, st) != 0) return -1;
        }
        {
            Tick tk(m, GV_K_COMBINE, st);
            hipLaunchKernelGGL(combine_kernel, dim3(M, (H + 255) / 256), dim3(256), 0, st, m.y, H, c.top_k, m.route + l,
                               m.sp, m.x);
        }
    }
    {
            Tick tk(m, GV_K_QUANT, st);
            if (quantize_act(m.x, H, M, H, m.final_norm, c.eps, 0, m.act_h, abH, nullptr, 0, st) != 0) return -1;
        }
    {
            Tick tk(m, GV_K_LM_HEAD, st);
            if (gemv_q4(m.lm_head, m.act_h, abH, M, gemv_out(m.logits, c.vocab, m.lm_head.global), st) != 0) return -1;
        }
    GV_CHECK_HIP(hipGetLastError());
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

int64_t qkv_rows(const gv_model_config &c) {
    return static_cast<int64_t>(c.n_heads) * 2 * c.head_dim + 2 * static_cast<int64_t>(c.n_kv_heads) * c.head_dim;
}

}  // namespace

}  // namespace gv

using namespace gv;

struct gv_model {
    Model m;
    std::vector<uint8_t *> staging;   // device staging, freed at the end of the call that made it
};

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
    auto fail = [&](const std::string &msg) -> gv_model * {
        put_err(err, err_len, msg);
        set_error(msg);
        return nullptr;
    };
    if (c.hidden <= 0 || c.hidden % 128 != 0) return fail("hidden must be a positive multiple of 128");
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
    if (c.vocab <= 0 || c.n_layers <= 0 || c.max_ctx <= c.max_rows) return fail("vocab, n_layers, max_ctx");
    {
        int waves, kw;
        const int ntt = c.max_rows <= 16 ? 1 : 2;
        if (!mfma_split(c.hidden, ntt, waves, kw) || !mfma_split(c.moe_ff, ntt, waves, kw))
            return fail("the expert products take hidden and moe_ff up to 4096 (2048 when max_rows > 16)");
    }
    auto g = std::make_unique<gv_model>();
    Model &m = g->m;
    m.c = c;
    m.E1 = c.n_experts + 1;
    const int64_t H = c.hidden, F = c.moe_ff, V = c.vocab, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    m.gu_code_stride = q4_code_bytes(2 * F, H);
    m.gu_scale_stride = q4_scale_bytes(2 * F, H);
    m.dn_code_stride = q4_code_bytes(H, F);
    m.dn_scale_stride = q4_scale_bytes(H, F);
    const int64_t kv_row = nkv * hd;
    bool ok = alloc_q4(m, m.embed, V, H) && alloc_q4(m, m.lm_head, V, H);
    ok = ok && (m.final_norm = static_cast<float *>(dalloc(m, H * 4)));
    m.slots = (static_cast<int64_t>(c.max_ctx) + kAttnBlock - 1) / kAttnBlock * kAttnBlock;
    const size_t kv_layer = 2 * static_cast<size_t>(nkv) * m.slots * hd;   // halves
    m.kv_all = static_cast<_Float16 *>(dalloc(m, static_cast<size_t>(c.n_layers) * kv_layer * 2));
    ok = ok && m.kv_all;
    m.layers.resize(static_cast<size_t>(c.n_layers));
    for (int l = 0; ok && l < c.n_layers; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        ok = alloc_q4(m, L.qkv, qkv_rows(c), H) && alloc_q4(m, L.o, H, nh * hd);
        auto *f = static_cast<float *>(dalloc(m, (2 * H + 2 * hd) * 4));
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
        L.kv = m.kv_all + static_cast<size_t>(l) * kv_layer;
    }
    const int Mx = c.max_rows, K = c.top_k;
    m.max_slots = std::min(c.n_experts, Mx * K) + 1;
    m.max_picks = Mx * (K + 1);
    m.kv_blocks = (c.max_ctx + kAttnBlock - 1) / kAttnBlock;
    ok = ok && (m.sp = static_cast<StepParams *>(dalloc(m, sizeof(StepParams))));
    ok = ok && (m.route = static_cast<RouteState *>(dalloc(m, sizeof(RouteState) * c.n_layers)));
    ok = ok && (m.x = static_cast<float *>(dalloc(m, Mx * H * 4)));
    ok = ok && (m.h = static_cast<float *>(dalloc(m, Mx * H * 4)));
    ok = ok && (m.qkv_out = static_cast<float *>(dalloc(m, Mx * qkv_rows(c) * 4)));
    ok = ok && (m.q16 = static_cast<_Float16 *>(dalloc(m, 2 * Mx * nh * hd * 2)));
    ok = ok && (m.core = static_cast<float *>(dalloc(m, Mx * nh * hd * 4)));
    ok = ok && (m.rlogits = static_cast<float *>(dalloc(m, Mx * m.E1 * 4)));
    ok = ok && (m.parts = static_cast<float *>(dalloc(m, static_cast<size_t>(Mx) * nh * m.kv_blocks * (hd + 2) * 4)));
    ok = ok && (m.gu_out = static_cast<float *>(dalloc(m, static_cast<size_t>(m.max_picks) * 2 * F * 4)));
    ok = ok && (m.y = static_cast<float *>(dalloc(m, static_cast<size_t>(m.max_picks) * H * 4)));
    ok = ok && (m.logits = static_cast<float *>(dalloc(m, static_cast<size_t>(Mx) * V * 4)));
    ok = ok && (m.act_h = static_cast<_Float16 *>(dalloc(m, Mx * act_bytes(H))));
    ok = ok && (m.act_core = static_cast<_Float16 *>(dalloc(m, Mx * act_bytes(nh * hd))));
    ok = ok && (m.act_m = static_cast<_Float16 *>(dalloc(m, m.max_picks * act_bytes(F))));
    ok = ok && (m.route_ids = static_cast<int32_t *>(dalloc(m, static_cast<size_t>(c.n_layers) * Mx * K * 4)));
    const int half = c.rope_dim / 2;
    const int npos = c.max_ctx + kMaxRows;
    ok = ok && (m.rope_cos = static_cast<float *>(dalloc(m, static_cast<size_t>(npos) * std::max(1, half) * 4)));
    ok = ok && (m.rope_sin = static_cast<float *>(dalloc(m, static_cast<size_t>(npos) * std::max(1, half) * 4)));
    if (!ok) {
        for (void *p : m.allocs) (void)hipFree(p);
        m.allocs.clear();
        return fail("gv_model_create: out of device memory");
    }
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
    if (hipMemset(m.kv_all, 0, static_cast<size_t>(c.n_layers) * kv_layer * 2) != hipSuccess)
        return fail("gv_model_create: memset failed");
    return g.release();
}

void gv_model_free(gv_model *g) {
    if (!g) return;
    (void)hipStreamSynchronize(stream());
    for (void *p : g->m.allocs) (void)hipFree(p);
    delete g;
}

int gv_model_adopt(gv_model *g, int kind, int layer, int expert, const void *data, int64_t bytes,
                   const float *globals) {
    GV_REQUIRE(g && data, "gv_model_adopt: null pointer");
    Model &m = g->m;
    const auto &c = m.c;
    const int64_t H = c.hidden, F = c.moe_ff, V = c.vocab, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const bool per_layer = kind != GV_EMBED && kind != GV_LM_HEAD && kind != GV_FINAL_NORM;
    GV_REQUIRE(!per_layer || (layer >= 0 && layer < c.n_layers), "gv_model_adopt: no such layer");
    LayerW *L = per_layer ? &m.layers[static_cast<size_t>(layer)] : nullptr;
    auto q4_size = [](int64_t r, int64_t cc) { return r * (cc / 16) * 9; };
    auto copy = [&](void *dst, int64_t want) -> int {
        GV_REQUIRE(bytes == want, "gv_model_adopt: wrong size for this tensor");
        GV_CHECK_HIP(hipMemcpy(dst, data, static_cast<size_t>(bytes), hipMemcpyHostToDevice));
        return 0;
    };
    switch (kind) {
    case GV_EMBED:
    case GV_LM_HEAD: {
        GV_REQUIRE(globals && bytes == q4_size(V, H), "gv_model_adopt: embed / lm_head size");
        Q4 &q = kind == GV_EMBED ? m.embed : m.lm_head;
        return upload_q4(data, false, V, H, const_cast<uint8_t *>(q.codes), const_cast<uint8_t *>(q.scales),
                         globals[0], q);
    }
    case GV_FINAL_NORM: return copy(m.final_norm, H * 4);
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
        std::vector<float> f(static_cast<size_t>(2 * n * kv_row));
        const auto *hsrc = static_cast<const uint16_t *>(data);
        for (size_t i = 0; i < f.size(); ++i) f[i] = static_cast<float>(__builtin_bit_cast(_Float16, hsrc[i]));
        float *dsrc = nullptr;
        GV_CHECK_HIP(hipMalloc(&dsrc, f.size() * 4 + 4));
        GV_CHECK_HIP(hipMemcpy(dsrc, f.data(), f.size() * 4, hipMemcpyHostToDevice));
        hipLaunchKernelGGL(kv_from_rows_kernel, dim3(static_cast<unsigned>((f.size() + 255) / 256)), dim3(256), 0,
                           stream(), dsrc, static_cast<int>(n), static_cast<int>(nkv), static_cast<int>(hd), m.slots, L->kv);
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
                                               static_cast<int64_t>(m.E1) * H});
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
    for (int l = 0; l < c.n_layers && rc == 0; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        rc |= make_f32(tseed(GV_IN_NORM, l, 0), H, 0.02f, L.in_norm);
        rc |= make_f32(tseed(GV_POST_NORM, l, 0), H, 0.02f, L.post_norm);
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
        if (ctx > 0) {   // K then V of positions [0, ctx) in the reference's row layout, then the device's
            for (int kvi = 0; kvi < 2; ++kvi)
                rc |= fill_normal(tseed(GV_KV, l, kvi), static_cast<int64_t>(ctx) * kv_row, 1.0f,
                                  wf + static_cast<int64_t>(kvi) * ctx * kv_row, st);
            hipLaunchKernelGGL(kv_from_rows_kernel, dim3(static_cast<unsigned>((2 * ctx * kv_row + 255) / 256)), dim3(256),
                               0, st, wf, ctx, static_cast<int>(nkv), static_cast<int>(hd), m.slots, L.kv);
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
    return 0;
}

int gv_model_set_position(gv_model *g, int pos) {
    GV_REQUIRE(g && pos >= 0 && pos + g->m.c.max_rows <= g->m.c.max_ctx, "gv_model_set_position: out of range");
    g->m.pos = pos;
    g->m.last_n = 0;
    return 0;
}

int gv_model_position(const gv_model *g) { return g ? g->m.pos : -1; }

int gv_verify(gv_model *g, const int32_t *tokens, int n, const int32_t *parents, float *logits) {
    GV_REQUIRE(g && tokens, "gv_verify: null pointer");
    Model &m = g->m;
    const auto &c = m.c;
    GV_REQUIRE(n >= 1 && n <= c.max_rows, "gv_verify: 1 <= n <= max_rows");
    GV_REQUIRE(m.pos + n <= c.max_ctx, "gv_verify: the context is full");
    StepParams &sp = m.host_sp;
    std::memset(&sp, 0, sizeof sp);
    sp.pos = m.pos;
    sp.M = n;
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
    hipStream_t st = stream();
    GV_CHECK_HIP(hipMemcpyAsync(m.sp, &sp, sizeof sp, hipMemcpyHostToDevice, st));
    if (run_layers(m, n, st) != 0) return -1;
    if (logits) {
        GV_CHECK_HIP(hipMemcpyAsync(logits, m.logits, static_cast<size_t>(n) * c.vocab * 4, hipMemcpyDeviceToHost, st));
        GV_CHECK_HIP(hipStreamSynchronize(st));
    }
    m.last_pos = m.pos;
    m.last_n = n;
    m.pos += n;
    return 0;
}

int gv_verify_keep(gv_model *g, int kept, const int32_t *path) {
    GV_REQUIRE(g, "gv_verify_keep: null model");
    Model &m = g->m;
    GV_REQUIRE(m.last_n > 0 && m.pos == m.last_pos + m.last_n, "gv_verify_keep: no verify to keep from");
    GV_REQUIRE(kept >= 1 && kept <= m.last_n, "gv_verify_keep: 1 <= kept <= n");
    if (path) {
        GV_REQUIRE(path[0] == 0, "gv_verify_keep: the path starts at the root (row 0)");
        for (int j = 1; j < kept; ++j) GV_REQUIRE(path[j] > path[j - 1] && path[j] < m.last_n, "gv_verify_keep: path");
        int *dpath = reinterpret_cast<int *>(m.rlogits);   // scratch: free between verifies
        GV_CHECK_HIP(hipMemcpyAsync(dpath, path, static_cast<size_t>(kept) * 4, hipMemcpyHostToDevice, stream()));
        const int64_t n = static_cast<int64_t>(m.c.n_layers) * m.c.n_kv_heads * m.c.head_dim;
        hipLaunchKernelGGL(kv_compact_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream(),
                           m.kv_all, m.c.n_layers, m.c.n_kv_heads, m.c.head_dim, m.slots, m.last_pos, kept, dpath);
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipStreamSynchronize(stream()));
    }
    m.pos = m.last_pos + kept;
    m.last_n = 0;
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
