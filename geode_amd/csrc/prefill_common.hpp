// The prefill MoE's (C5) device code shared by its separate launches (model.hip) and its fused ones (prefill.hip):
// the shared expert's gate logits and the placement of one expert's picks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gv {

// The shared expert's gate logit of row t: the bf16 row . h in the router's eight-sum order (bf16_row_dots,
// kernels.cpp:1446-1483); a wave a row, 4 rows a workgroup of 256 threads. gr_lds: the gate row as fp32 [H], then the
// waves' rows [4][H]. Every global load is issued before the first store to the LDS (the gate row 8 values a thread,
// the wave's row 4 values a lane, 2048 values a pass), then the eight fixed-order chains run from the LDS. Every
// thread calls this (one barrier); the logit is lane 0's, for t < M.
__device__ inline float gate_row_logit(const uint16_t *__restrict__ wrow, int H, const float *__restrict__ h, int M,
                                       int t, float *gr_lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *ws = gr_lds, *hs = gr_lds + H + wave * H;
    const float *hr = h + static_cast<int64_t>(min(t, M - 1)) * H;
    for (int p0 = 0; p0 < H; p0 += 2048) {
        uint4 wv = make_uint4(0, 0, 0, 0);
        const int iw = p0 + static_cast<int>(threadIdx.x) * 8;
        if (iw < H) wv = *reinterpret_cast<const uint4 *>(wrow + iw);
        float4 hv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int ih = min(p0 + u * 256 + lane * 4, H - 4);
            hv[u] = *reinterpret_cast<const float4 *>(hr + ih);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (iw < H) {
            const uint32_t wu[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ws[iw + 2 * k] = __uint_as_float(wu[k] << 16);
                ws[iw + 2 * k + 1] = __uint_as_float(wu[k] & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int ih = p0 + u * 256 + lane * 4;
            if (ih < H) *reinterpret_cast<float4 *>(hs + ih) = hv[u];
        }
    }
    __syncthreads();
    if (t >= M) return 0.0f;
    float a = 0.0f;
    if (lane < 8)
        for (int c0 = lane; c0 < H; c0 += 8 * 16) {   // 16 steps' operands read ahead of their sums
            float hv[16], wv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                hv[u] = hs[c0 + 8 * u];
                wv[u] = ws[c0 + 8 * u];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) a = __fadd_rn(a, __fmul_rn(wv[u], hv[u]));
        }
    const float s1 = __fadd_rn(a, __shfl_down(a, 4, 64));   // ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7))
    const float s2 = __fadd_rn(s1, __shfl_down(s1, 1, 64));
    const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));
    return s3;
}

// The picks of expert e in (token, rank) order, by ordered compaction over ids [M][K] (e's first pick at s0): their
// rows and, per (row, rank), where the pick went; the shared expert (E) takes row t at s0 + t. A workgroup of 256
// threads calls this; wt: LDS of kFillBatch x 4 ints.
constexpr int kFillBatch = 16;
__device__ inline void fill_expert_picks(const int *__restrict__ ids, int M, int K, int E, int e, int s0,
                                         int *__restrict__ pick_token, int *__restrict__ pick_of,
                                         int (*wt)[4]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (e == E) {
        for (int t = tid; t < M; t += blockDim.x) {
            pick_token[s0 + t] = t;
            pick_of[t * (K + 1) + K] = s0 + t;
        }
        return;
    }
    // kFillBatch chunks of 256 ids at a time: every id of the batch loaded at once, each chunk's matches counted per
    // wave, one barrier, then each match placed after the earlier chunks' and waves' (the same order as one chunk at
    // a time)
    int base = 0;
    for (int c0 = 0; c0 < M * K; c0 += kFillBatch * 256) {
        int idv[kFillBatch];
#pragma unroll
        for (int u = 0; u < kFillBatch; ++u) idv[u] = ids[min(c0 + u * 256 + tid, M * K - 1)];
        uint64_t bal[kFillBatch];
#pragma unroll
        for (int u = 0; u < kFillBatch; ++u) {
            bal[u] = __ballot(c0 + u * 256 + tid < M * K && idv[u] == e);
            if (lane == 0) wt[u][wave] = __popcll(bal[u]);
        }
        __syncthreads();
        int run = base;
#pragma unroll
        for (int u = 0; u < kFillBatch; ++u) {
            int wb = run;
            for (int w2 = 0; w2 < wave; ++w2) wb += wt[u][w2];
            if ((bal[u] >> lane) & 1ull) {
                const int i = c0 + u * 256 + tid;
                const int p = s0 + wb + __popcll(bal[u] & ((1ull << lane) - 1ull)), t = i / K, k = i % K;
                pick_token[p] = t;
                pick_of[t * (K + 1) + k] = p;
            }
            run += wt[u][0] + wt[u][1] + wt[u][2] + wt[u][3];
        }
        base = run;
        __syncthreads();   // (wt is the next batch's)
    }
}

}  // namespace gv
