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

#include "gemv_core.hpp"
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
    const int nch = static_cast<int>(w.cols / 32), groups = q4_groups(w.steps);
    for (int c = threadIdx.x; c < nch; c += blockDim.x) {
        const uint4 cw = *reinterpret_cast<const uint4 *>(w.codes + q4_code_offset(w.rows, w.cols, w.S, r, c));
        const uint8_t *sd = w.scales + q4_scale_offset(w.rows, w.S, groups, r, c);
        const uint32_t words[4] = {cw.x, cw.y, cw.z, cw.w};
        float *o = x + static_cast<int64_t>(t) * w.cols + c * 32;
        for (int j = 0; j < 2; ++j) {
            const float s = __fmul_rn(e4m3_to_f32(sd[j]), w.global);
            for (int q = 0; q < 2; ++q)
                for (int b = 0; b < 8; ++b) {
                    const int cp = static_cast<int>((words[2 * j + q] >> (4 * b)) & 15u);
                    o[16 * j + 8 * q + b] = __fmul_rn(static_cast<float>(2 * cp - 15), s);
                }
        }
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

// Per (row, head): the query heads' and key heads' RMSNorm(1 + w) then partial RoPE on the first rope_dim dims
// (pairs i, i + half; model.cpp:3714-3733, rotary position pos + depth), the keys and values appended to the fp16
// cache at slot pos + row (static_cast<_Float16>: round to nearest even). Query heads go to q_out [M][nh][hd].
__global__ __launch_bounds__(256) void qk_rope_kernel(const float *__restrict__ qkv, int64_t ldq, int nh, int nkv, int hd,
                                                      int half, const float *__restrict__ q_norm,
                                                      const float *__restrict__ k_norm, float eps,
                                                      const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                                      const StepParams *__restrict__ sp, float *__restrict__ q_out,
                                                      uint16_t *__restrict__ kv, int max_ctx) {
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
        if (i < hd) kv[(static_cast<int64_t>(max_ctx) + slot) * kv_row + kh * hd + i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(xv));
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
    if (kind == 0) q_out[(static_cast<int64_t>(t) * nh + head) * hd + i] = out;
    else kv[static_cast<int64_t>(slot) * kv_row + kh * hd + i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(out));
}

// Split-KV attention (flash decoding over blocks of kAttnBlock positions): a workgroup per (block, KV head) takes the
// group of query heads that share the KV head for every row; scores q.k / sqrt(hd) (eight partial sums in the
// reference's order, model.cpp:3927-3948), masked to the context plus the row's visible rows, the block's maximum,
// exp(score - max), their sum and the weighted values: parts [M][nh][blocks][hd + 2] (model.cpp:3990-4018).
__global__ __launch_bounds__(256) void attn_part_kernel(const float *__restrict__ q_out, const uint16_t *__restrict__ kv,
                                                        int max_ctx, int nh, int nkv, int hd,
                                                        const StepParams *__restrict__ sp, float *__restrict__ parts,
                                                        int nb_max) {
    extern __shared__ uint4 lds_u4[];
    const int b = blockIdx.x, kh = blockIdx.y;
    const int pos = sp->pos, M = sp->M, total = pos + M;
    const int s0 = b * kAttnBlock;
    if (s0 >= total) return;
    const int ns = min(kAttnBlock, total - s0);
    const int group = nh / nkv, NQ = group * M;
    const int64_t kv_row = static_cast<int64_t>(nkv) * hd;
    uint16_t *Kt = reinterpret_cast<uint16_t *>(lds_u4);
    uint16_t *Vt = Kt + kAttnBlock * hd;
    float *Qc = reinterpret_cast<float *>(Vt + kAttnBlock * hd);   // [16][hd]
    float *Sc = Qc + 16 * hd;                                       // [16][kAttnBlock]
    for (int idx = threadIdx.x; idx < ns * hd; idx += blockDim.x) {
        const int s = idx / hd, d = idx % hd;
        Kt[idx] = kv[static_cast<int64_t>(s0 + s) * kv_row + kh * hd + d];
        Vt[idx] = kv[(static_cast<int64_t>(max_ctx) + s0 + s) * kv_row + kh * hd + d];
    }
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(hd)));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int qc = 0; qc < NQ; qc += 16) {
        const int nq = min(16, NQ - qc);
        __syncthreads();
        for (int idx = threadIdx.x; idx < nq * hd; idx += blockDim.x) {
            const int j = idx / hd, d = idx % hd, qi = qc + j;
            const int t = qi / group, h = kh * group + qi % group;
            Qc[idx] = q_out[(static_cast<int64_t>(t) * nh + h) * hd + d];
        }
        __syncthreads();
        for (int pr = threadIdx.x; pr < nq * ns; pr += blockDim.x) {
            const int j = pr / ns, s = pr % ns, slot = s0 + s, t = (qc + j) / group;
            const bool visible = slot < pos || ((sp->vis[t] >> (slot - pos)) & 1u);
            float sv = -__builtin_inff();
            if (visible) {
                float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                const float *q = Qc + j * hd;
                const uint16_t *k = Kt + s * hd;
                for (int d = 0; d < hd; d += 8)
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        acc[u] = __fadd_rn(acc[u], __fmul_rn(q[d + u], static_cast<float>(__builtin_bit_cast(_Float16, k[d + u]))));
                const float dot = __fadd_rn(__fadd_rn(__fadd_rn(acc[0], acc[4]), __fadd_rn(acc[1], acc[5])),
                                            __fadd_rn(__fadd_rn(acc[2], acc[6]), __fadd_rn(acc[3], acc[7])));
                sv = __fmul_rn(dot, scale);
            }
            Sc[j * kAttnBlock + s] = sv;
        }
        __syncthreads();
        __shared__ float ml[16][2];
        for (int j = wave; j < nq; j += 4) {
            const float sv = lane < ns ? Sc[j * kAttnBlock + lane] : -__builtin_inff();
            const float mx = wave_max(sv);
            const float e = (sv == -__builtin_inff()) ? 0.0f : expf(__fsub_rn(sv, mx));
            float l = e;
            for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
            if (lane < ns) Sc[j * kAttnBlock + lane] = e;
            if (lane == 0) {
                ml[j][0] = mx;
                ml[j][1] = l;
            }
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < nq * hd; idx += blockDim.x) {
            const int j = idx / hd, d = idx % hd, qi = qc + j;
            const int t = qi / group, h = kh * group + qi % group;
            float o = 0.0f;
            for (int s = 0; s < ns; ++s)
                o = __builtin_fmaf(Sc[j * kAttnBlock + s], static_cast<float>(__builtin_bit_cast(_Float16, Vt[s * hd + d])), o);
            float *dst = parts + ((static_cast<int64_t>(t) * nh + h) * nb_max + b) * (hd + 2);
            dst[d] = o;
            if (d == 0) {
                dst[hd] = ml[j][0];
                dst[hd + 1] = ml[j][1];
            }
        }
    }
}

// The blocks joined per (row, head): exp(block max - max), the sums, 1 / sum, times sigmoid(gate)
// (model.cpp:3830-3855); the row's core then quantized for o_proj.
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ parts, const float *__restrict__ qkv,
                                                         int64_t ldq, int nh, int hd, int nb_max,
                                                         const StepParams *__restrict__ sp, float *__restrict__ core,
                                                         uint8_t *__restrict__ act_core, int64_t act_stride) {
    extern __shared__ uint4 lds_u4[];
    float *row = reinterpret_cast<float *>(lds_u4);
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const int nbw = (sp->pos + sp->M + kAttnBlock - 1) / kAttnBlock;
    for (int idx = threadIdx.x; idx < nh * hd; idx += blockDim.x) {
        const int h = idx / hd, d = idx % hd;
        const float *base = parts + ((static_cast<int64_t>(t) * nh + h) * nb_max) * (hd + 2);
        float mx = -__builtin_inff();
        for (int b = 0; b < nbw; ++b) mx = fmaxf(mx, base[b * (hd + 2) + hd]);
        float o = 0.0f, l = 0.0f;
        for (int b = 0; b < nbw; ++b) {
            const float *pb = base + b * (hd + 2);
            const float f = pb[hd] == -__builtin_inff() ? 0.0f : expf(__fsub_rn(pb[hd], mx));
            l = __fadd_rn(l, __fmul_rn(pb[hd + 1], f));
            o = __fadd_rn(o, __fmul_rn(pb[d], f));
        }
        const float gate = qkv[t * ldq + static_cast<int64_t>(h) * 2 * hd + hd + d];
        const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gate)));
        const float val = __fmul_rn(__fmul_rn(o, __fdiv_rn(1.0f, l)), sig);
        row[idx] = val;
        core[static_cast<int64_t>(t) * nh * hd + idx] = val;
    }
    __syncthreads();
    quantize_row(row, nh * hd, act_core + t * act_stride);
}

// Router logits: bf16 rows [E + 1][H] (the shared expert's gate row last) times the post-norm rows, eight partial
// sums per row in the reference's fixed order (bf16_row_dots, kernels.cpp:1446-1483). A wave per row, its lanes
// 8 tokens x 8 partial sums.
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
        float acc = 0.0f;
        if (t < M) {
            const float *x = h + static_cast<int64_t>(t) * H;
            for (int c = 0; c < H; c += 8) {
                const float wf = __uint_as_float(static_cast<uint32_t>(row[c + j]) << 16);
                acc = __fadd_rn(acc, __fmul_rn(wf, x[c + j]));
            }
        }
        const float s = __fadd_rn(acc, __shfl_down(acc, 4, 64));          // lanes j < 4: a_j + a_{j+4}
        const float s2 = __fadd_rn(s, __shfl_down(s, 1, 64));             // j = 0: s0 + s1, j = 2: s2 + s3
        const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));           // j = 0: (s0 + s1) + (s2 + s3)
        if (j == 0 && t < M) logits[static_cast<int64_t>(t) * E1 + r] = s3;
    }
}

// The route (route_topk, model.cpp:4021-4065): softmax over the experts (max, expf, the sum in index order, divide),
// the top K by probability with ties to the lower index, the weights p / (their sum in rank order); the shared
// expert's gate sigmoid(logit); then the slots (distinct experts ascending, the shared one last) and their picks.
__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ logits, int E, int K,
                                                    const StepParams *__restrict__ sp, RouteState *__restrict__ rs,
                                                    int32_t *__restrict__ ids_out) {
    __shared__ float p[kMaxRows][256];
    __shared__ int ids[kMaxRows * 16];
    __shared__ int cursor[257];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int M = sp->M, E1 = E + 1;
    for (int t = wave; t < M; t += 4) {
        const float *lg = logits + static_cast<int64_t>(t) * E1;
        float mx = -__builtin_inff();
        for (int e = lane; e < E; e += 64) mx = fmaxf(mx, lg[e]);
        mx = wave_max(mx);
        for (int e = lane; e < E; e += 64) p[t][e] = expf(__fsub_rn(lg[e], mx));
        __builtin_amdgcn_wave_barrier();
        float sum = 0.0f;
        if (lane == 0)
            for (int e = 0; e < E; ++e) sum = __fadd_rn(sum, p[t][e]);
        sum = __shfl(sum, 0, 64);
        for (int e = lane; e < E; e += 64) p[t][e] = __fdiv_rn(p[t][e], sum);
        __builtin_amdgcn_wave_barrier();
        float top = 0.0f;
        float pk[16];
        for (int k = 0; k < K; ++k) {
            float bv = -1.0f;
            int bi = E;
            for (int e = lane; e < E; e += 64) {
                bool taken = false;
                for (int q = 0; q < k; ++q) taken |= ids[t * 16 + q] == e;
                const float v = p[t][e];
                if (!taken && (v > bv || (v == bv && e < bi))) bv = v, bi = e;
            }
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) bv = ov, bi = oi;
            }
            if (lane == 0) ids[t * 16 + k] = bi;
            __builtin_amdgcn_wave_barrier();
            pk[k] = bv;
            top = __fadd_rn(top, bv);
        }
        if (lane < K) {
            float mine = 0.0f;
            for (int k = 0; k < K; ++k)
                if (k == lane) mine = pk[k];
            rs->weight[t * K + lane] = __fdiv_rn(mine, top);
            ids_out[t * K + lane] = ids[t * 16 + lane];
        }
        if (lane == 0) rs->gate[t] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-lg[E])));
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int e = 0; e <= E; ++e) cursor[e] = 0;
    for (int t = 0; t < M; ++t)
        for (int k = 0; k < K; ++k) ++cursor[ids[t * 16 + k]];
    cursor[E] = M;
    int u = 0, run = 0;
    for (int e = 0; e <= E; ++e) {
        const int c = cursor[e];
        cursor[e] = run;
        if (c > 0) {
            rs->slot_expert[u] = e;
            rs->slot_start[u] = run;
            rs->slot_count[u] = c;
            ++u;
        }
        run += c;
    }
    rs->n_slots = u;
    rs->n_picks = run;
    for (int t = 0; t < M; ++t) {
        for (int k = 0; k < K; ++k) {
            const int pk_ = cursor[ids[t * 16 + k]]++;
            rs->pick_token[pk_] = t;
            rs->pick_of[t * (K + 1) + k] = pk_;
        }
        const int ps = cursor[E]++;
        rs->pick_token[ps] = t;
        rs->pick_of[t * (K + 1) + K] = ps;
    }
}

// The experts' products, a workgroup per (slot, row tile): UP takes gate_up [2F x H] against the post-norm rows of
// the slot's tokens, DOWN takes down [H x F] against the slot's picks' SwiGLU rows; each pick's rows go to out.
template <int S, int R, int MT, bool UP>
__global__ __launch_bounds__(256) void moe_gemv_kernel(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales,
                                                       size_t code_stride, size_t scale_stride, int64_t rows,
                                                       int64_t cols, int steps, const float *__restrict__ globals,
                                                       int half_rows, const uint8_t *__restrict__ act,
                                                       const RouteState *__restrict__ rs, float *__restrict__ out) {
    constexpr int G = 64 / S;
    constexpr int WROWS = G * R;
    extern __shared__ uint4 lds_u4[];
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds_u4);
    const int u = blockIdx.x;
    if (u >= rs->n_slots) return;
    const int e = rs->slot_expert[u], start = rs->slot_start[u], cnt = rs->slot_count[u];
    const int64_t abytes = (cols / 32) * kActChunkBytes;
    for (int64_t i = static_cast<int64_t>(threadIdx.x) * 16; i < cnt * abytes; i += static_cast<int64_t>(blockDim.x) * 16) {
        const int64_t j = i / abytes, o = i % abytes;
        const int64_t src_row = UP ? rs->pick_token[start + j] : start + j;
        *reinterpret_cast<uint4 *>(lds + i) = *reinterpret_cast<const uint4 *>(act + src_row * abytes + o);
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane / S, k = lane % S;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.y) * 4 + wave) * WROWS;
    if (row0 >= rows) return;
    float acc[R][MT];
    gemv_wave<S, R, MT>(codes + static_cast<size_t>(e) * code_stride, scales + static_cast<size_t>(e) * scale_stride,
                        rows, cols, steps, row0, lds, abytes, cnt, g, k, acc);
    gemv_reduce<S, R, MT>(acc, cnt);
    if (k != 0) return;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int64_t row = row0 + i * G + g;
        if (row >= rows) continue;
        const float gl = UP ? (row < half_rows ? globals[e * 3] : globals[e * 3 + 1]) : globals[e * 3 + 2];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= cnt) break;
            out[static_cast<int64_t>(start + t) * rows + row] = acc[i][t] * gl;
        }
    }
}

// per pick: silu(gate) * up (kernels.hpp:141), quantized for down
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float *__restrict__ gu, int F,
                                                           const RouteState *__restrict__ rs,
                                                           uint8_t *__restrict__ act_m) {
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
    quantize_row(m, F, act_m + static_cast<int64_t>(p) * (F / 32) * kActChunkBytes);
}

// x += sigmoid(gate) x shared + sum_k w_k y_k in rank order (model.cpp:4554-4585, :5363-5365)
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ y, int H, int K,
                                                      const RouteState *__restrict__ rs,
                                                      const StepParams *__restrict__ sp, float *__restrict__ x) {
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const float gs = rs->gate[t];
    const float *sh = y + static_cast<int64_t>(rs->pick_of[t * (K + 1) + K]) * H;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float o = __fmul_rn(gs, sh[i]);
        for (int k = 0; k < K; ++k) {
            const float wk = rs->weight[t * K + k];
            if (wk == 0.0f) continue;
            o = __fadd_rn(o, __fmul_rn(wk, y[static_cast<int64_t>(rs->pick_of[t * (K + 1) + k]) * H + i]));
        }
        x[static_cast<int64_t>(t) * H + i] = __fadd_rn(x[static_cast<int64_t>(t) * H + i], o);
    }
}

// verify_keep of a tree: the kept path's KV rows moved to the kept slots in every layer
__global__ void kv_compact_kernel(uint16_t *kv_all, int n_layers, int max_ctx, int64_t kv_row, int pos, int kept,
                                  const int *__restrict__ path) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t per_layer = 2 * kv_row;
    if (i >= n_layers * per_layer) return;
    const int l = static_cast<int>(i / per_layer), kvi = static_cast<int>((i % per_layer) / kv_row);
    const int64_t d = i % kv_row;
    uint16_t *base = kv_all + (static_cast<int64_t>(l) * 2 + kvi) * max_ctx * kv_row;
    for (int j = 1; j < kept; ++j)   // ascending: path[j] >= j, so no source is overwritten before it is read
        if (path[j] != j) base[(pos + j) * kv_row + d] = base[(pos + path[j]) * kv_row + d];
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

template <int S, int R, int MT, bool UP>
int launch_moe(const Model &m, const LayerW &L, int M, hipStream_t st) {
    constexpr int WROWS = (64 / S) * R;
    const int64_t H = m.c.hidden, F = m.c.moe_ff;
    const int64_t rows = UP ? 2 * F : H, cols = UP ? H : F;
    const int steps = static_cast<int>(cols / (32 * S));
    const int tiles = static_cast<int>((rows + 4 * WROWS - 1) / (4 * WROWS));
    const size_t lds = static_cast<size_t>(M) * act_bytes(cols);
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&moe_gemv_kernel<S, R, MT, UP>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL((moe_gemv_kernel<S, R, MT, UP>), dim3(m.max_slots, tiles), dim3(256), lds, st,
                       UP ? L.gu_codes : L.dn_codes, UP ? L.gu_scales : L.dn_scales,
                       UP ? m.gu_code_stride : m.dn_code_stride, UP ? m.gu_scale_stride : m.dn_scale_stride, rows, cols,
                       steps, L.expert_globals, static_cast<int>(F), UP ? m.act_h : m.act_m, m.route + (&L - &m.layers[0]),
                       UP ? m.gu_out : m.y);
    return 0;
}

template <int S, bool UP>
int moe_dispatch(const Model &m, const LayerW &L, int M, hipStream_t st) {
    if (M <= 1) return launch_moe<S, 1, 1, UP>(m, L, M, st);
    if (M <= 2) return launch_moe<S, 1, 2, UP>(m, L, M, st);
    if (M <= 4) return launch_moe<S, 1, 4, UP>(m, L, M, st);
    if (M <= 8) return launch_moe<S, 1, 8, UP>(m, L, M, st);
    if (M <= 16) return launch_moe<S, 1, 16, UP>(m, L, M, st);
    return launch_moe<S, 1, 32, UP>(m, L, M, st);
}

int moe_products(const Model &m, const LayerW &L, int M, bool up, hipStream_t st) {
    const int S = q4_lanes_for(up ? m.c.hidden : m.c.moe_ff);
    switch (S * 2 + (up ? 1 : 0)) {
    case 2: return moe_dispatch<1, false>(m, L, M, st);
    case 3: return moe_dispatch<1, true>(m, L, M, st);
    case 4: return moe_dispatch<2, false>(m, L, M, st);
    case 5: return moe_dispatch<2, true>(m, L, M, st);
    case 8: return moe_dispatch<4, false>(m, L, M, st);
    case 9: return moe_dispatch<4, true>(m, L, M, st);
    case 16: return moe_dispatch<8, false>(m, L, M, st);
    case 17: return moe_dispatch<8, true>(m, L, M, st);
    default: set_error("moe: unsupported width"); return -1;
    }
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

int run_layers(Model &m, int M, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim;
    const int64_t abH = static_cast<int64_t>(act_bytes(H)), abC = static_cast<int64_t>(act_bytes(static_cast<int64_t>(nh) * hd));
    const size_t lds_attn = (2 * static_cast<size_t>(kAttnBlock) * hd) * 2 + 16 * static_cast<size_t>(hd) * 4 +
                            16 * static_cast<size_t>(kAttnBlock) * 4;
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&attn_part_kernel), lds_attn, granted) != 0) return -1;
    hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, st, m.embed, m.sp, m.x);
    for (int l = 0; l < c.n_layers; ++l) {
        LayerW &L = m.layers[static_cast<size_t>(l)];
        if (quantize_act(m.x, H, M, H, L.in_norm, c.eps, m.act_h, abH, nullptr, 0, st) != 0) return -1;
        if (gemv_q4(L.qkv, m.act_h, abH, M, qkv_out(m, L), st) != 0) return -1;
        hipLaunchKernelGGL(qk_rope_kernel, dim3(M, nh + 2 * nkv), dim3(256), 0, st, m.qkv_out, L.qkv.rows, nh, nkv, hd,
                           c.rope_dim / 2, L.q_norm, L.k_norm, c.eps, m.rope_cos, m.rope_sin, m.sp, m.q_out, L.kv,
                           c.max_ctx);
        hipLaunchKernelGGL(attn_part_kernel, dim3(m.kv_blocks, nkv), dim3(256), lds_attn, st, m.q_out, L.kv, c.max_ctx,
                           nh, nkv, hd, m.sp, m.parts, m.kv_blocks);
        hipLaunchKernelGGL(attn_merge_kernel, dim3(M), dim3(256), static_cast<size_t>(nh) * hd * 4, st, m.parts,
                           m.qkv_out, L.qkv.rows, nh, hd, m.kv_blocks, m.sp, m.core, m.act_core, abC);
        if (gemv_q4(L.o, m.act_core, abC, M, gemv_out(m.x, H, L.o.global, 1), st) != 0) return -1;
        if (quantize_act(m.x, H, M, H, L.post_norm, c.eps, m.act_h, abH, m.h, H, st) != 0) return -1;
        hipLaunchKernelGGL(router_kernel, dim3((m.E1 + 3) / 4), dim3(256), 0, st, L.router, m.E1, H, m.h, m.sp,
                           m.rlogits);
        hipLaunchKernelGGL(route_kernel, dim3(1), dim3(256), 0, st, m.rlogits, c.n_experts, c.top_k, m.sp, m.route + l,
                           m.route_ids + static_cast<int64_t>(l) * c.max_rows * c.top_k);
        if (moe_products(m, L, M, true, st) != 0) return -1;
        hipLaunchKernelGGL(swiglu_quant_kernel, dim3(m.max_picks), dim3(256), static_cast<size_t>(c.moe_ff) * 4, st,
                           m.gu_out, c.moe_ff, m.route + l, m.act_m);
        if (moe_products(m, L, M, false, st) != 0) return -1;
        hipLaunchKernelGGL(combine_kernel, dim3(M), dim3(256), 0, st, m.y, H, c.top_k, m.route + l, m.sp, m.x);
    }
    if (quantize_act(m.x, H, M, H, m.final_norm, c.eps, m.act_h, abH, nullptr, 0, st) != 0) return -1;
    if (gemv_q4(m.lm_head, m.act_h, abH, M, gemv_out(m.logits, c.vocab, m.lm_head.global), st) != 0) return -1;
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
    q.S = q4_lanes_for(cols);
    q.steps = static_cast<int>(cols / (32 * q.S));
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
    if (c.hidden <= 0 || c.hidden % 256 != 0) return fail("hidden must be a positive multiple of 256");
    if (c.moe_ff <= 0 || c.moe_ff % 64 != 0 || c.shared_ff != c.moe_ff)
        return fail("moe_ff must be a positive multiple of 64 and shared_ff equal to it");
    if (c.head_dim <= 0 || c.head_dim > 256 || c.head_dim % 8 != 0 || c.rope_dim > c.head_dim || c.rope_dim % 2)
        return fail("head_dim must be a multiple of 8 up to 256, rope_dim even and <= head_dim");
    if (c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads != 0 || (c.n_heads * c.head_dim) % 256 != 0)
        return fail("n_heads must be a multiple of n_kv_heads, n_heads x head_dim a multiple of 256");
    if (c.n_experts <= 0 || c.n_experts > 256 || c.top_k <= 0 || c.top_k > 16 || c.top_k > c.n_experts)
        return fail("1 <= top_k <= 16, top_k <= n_experts <= 256");
    if (c.max_rows <= 0 || c.max_rows > kMaxRows) return fail("max_rows must be 1..32");
    if (c.vocab <= 0 || c.n_layers <= 0 || c.max_ctx <= c.max_rows) return fail("vocab, n_layers, max_ctx");
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
    m.kv_all = static_cast<uint16_t *>(dalloc(m, static_cast<size_t>(c.n_layers) * 2 * c.max_ctx * kv_row * 2));
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
        L.kv = m.kv_all + static_cast<size_t>(l) * 2 * c.max_ctx * kv_row;
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
    ok = ok && (m.q_out = static_cast<float *>(dalloc(m, Mx * nh * hd * 4)));
    ok = ok && (m.core = static_cast<float *>(dalloc(m, Mx * nh * hd * 4)));
    ok = ok && (m.rlogits = static_cast<float *>(dalloc(m, Mx * m.E1 * 4)));
    ok = ok && (m.parts = static_cast<float *>(dalloc(m, static_cast<size_t>(Mx) * nh * m.kv_blocks * (hd + 2) * 4)));
    ok = ok && (m.gu_out = static_cast<float *>(dalloc(m, static_cast<size_t>(m.max_picks) * 2 * F * 4)));
    ok = ok && (m.y = static_cast<float *>(dalloc(m, static_cast<size_t>(m.max_picks) * H * 4)));
    ok = ok && (m.logits = static_cast<float *>(dalloc(m, static_cast<size_t>(Mx) * V * 4)));
    ok = ok && (m.act_h = static_cast<uint8_t *>(dalloc(m, Mx * act_bytes(H))));
    ok = ok && (m.act_core = static_cast<uint8_t *>(dalloc(m, Mx * act_bytes(nh * hd))));
    ok = ok && (m.act_m = static_cast<uint8_t *>(dalloc(m, m.max_picks * act_bytes(F))));
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
    if (hipMemset(m.kv_all, 0, static_cast<size_t>(c.n_layers) * 2 * c.max_ctx * kv_row * 2) != hipSuccess)
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
        for (int kvi = 0; kvi < 2; ++kvi)
            GV_CHECK_HIP(hipMemcpy(L->kv + static_cast<size_t>(kvi) * c.max_ctx * kv_row,
                                   static_cast<const uint8_t *>(data) + kvi * n * kv_row * 2,
                                   static_cast<size_t>(n * kv_row * 2), hipMemcpyHostToDevice));
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
        if (ctx > 0) {
            for (int kvi = 0; kvi < 2; ++kvi) {
                rc |= fill_normal(tseed(GV_KV, l, kvi), static_cast<int64_t>(ctx) * kv_row, 1.0f, wf, st);
                hipLaunchKernelGGL(f32_to_f16_kernel, dim3(static_cast<unsigned>((ctx * kv_row + 255) / 256)), dim3(256), 0,
                                   st, wf, static_cast<int64_t>(ctx) * kv_row,
                                   L.kv + static_cast<size_t>(kvi) * c.max_ctx * kv_row);
            }
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
        const int64_t kv_row = static_cast<int64_t>(m.c.n_kv_heads) * m.c.head_dim;
        const int64_t n = static_cast<int64_t>(m.c.n_layers) * 2 * kv_row;
        hipLaunchKernelGGL(kv_compact_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream(),
                           m.kv_all, m.c.n_layers, m.c.max_ctx, kv_row, m.last_pos, kept, dpath);
        GV_CHECK_HIP(hipGetLastError());
        GV_CHECK_HIP(hipStreamSynchronize(stream()));
    }
    m.pos = m.last_pos + kept;
    m.last_n = 0;
    return 0;
}

const float *gv_model_logits(const gv_model *g) { return g ? g->m.logits : nullptr; }

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
