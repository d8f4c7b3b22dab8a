// The prefill MoE's (C5) work before the experts' products, in two launches instead of five: the three per-row
// steps (the shared expert's gate, the route, the products' operands) as roles of one launch, then the grouping of
// the picks by expert with their placement. Each output is what the separate kernels (model.hip: gate_rows_kernel,
// route_rows_kernel, quantize_act_kernel, group_kernel, fill_picks_kernel) write, bit for bit; gv_model_set_fused(m,
// 0) runs those instead. The kernels live in this source file of their own so that the verify step's kernels keep
// their places in model.hip's code object.
#include <algorithm>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"
#include "prefill_common.hpp"

namespace gv {
namespace {

// Three roles that read only the rows h and their routed logits and write disjoint outputs (no hand-off), g =
// ceil(M / 4), 256 threads:
//   workgroups [0, g)           the shared expert's gate logits (gate_row_logit, 4 rows a workgroup) to logits [t][E]
//                               and sigmoid(logit) to gate [t] (route_rows' arithmetic, model.cpp:4021-4065);
//   workgroups [g, 2g)          the rows' top K and their weights (route_row, 4 rows a workgroup) on a copy of each
//                               row's E routed logits in LDS (the copy leaves out column E, which the first role
//                               writes; route_row's gate output goes to that LDS slot, unused);
//   workgroups [2g, 2g + M)     row t's operands for the products (norm_quant_row without a norm, quantize_act's).
__global__ __launch_bounds__(256) void prefill_front_kernel(const uint16_t *__restrict__ wrow, int H,
                                                            const float *__restrict__ h, int M, int E, int K,
                                                            float *__restrict__ logits, _Float16 *__restrict__ act,
                                                            int64_t act_stride, int *__restrict__ ids,
                                                            float *__restrict__ w, float *__restrict__ gate) {
    extern __shared__ float pf_lds[];
    __shared__ double red[16];
    const int g = (M + 3) / 4, b = static_cast<int>(blockIdx.x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, E1 = E + 1;
    if (b < g) {
        const int t = b * 4 + wave;
        const float s = gate_row_logit(wrow, H, h, M, t, pf_lds);
        if (t < M && lane == 0) {
            logits[static_cast<int64_t>(t) * E1 + E] = s;
            gate[t] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-s)));
        }
    } else if (b < 2 * g) {
        const int t = (b - g) * 4 + wave;
        if (t >= M) return;   // (no barrier below: a wave's own row)
        float *row = pf_lds + wave * (E1 + 3);
        const float *src = logits + static_cast<int64_t>(t) * E1;
        for (int i = lane; i < E; i += 64) row[i] = src[i];
        if (lane == 0) row[E] = 0.0f;
        // (one wave's LDS operations complete in order: route_row's reads see the copy)
        route_row(row, E, K, ids + static_cast<int64_t>(t) * K, w + static_cast<int64_t>(t) * K, &row[E]);
    } else {
        const int t = b - 2 * g;
        norm_quant_row(h + static_cast<int64_t>(t) * H, H, nullptr, 0.0f, act + static_cast<int64_t>(t) * act_stride,
                       nullptr, red);
    }
}

// The picks grouped by expert and placed, a workgroup (256 threads) per expert e in [0, E]: every expert's pick
// count into LDS (the shared expert E takes every row), e's first pick and first slot as the sums of the counts and
// of the slot counts below e (integers: any order), e's slots (runs of at most 32 picks) and its picks' places
// (fill_expert_picks); workgroup E also writes the totals. group_kernel and fill_picks_kernel's outputs.
__global__ __launch_bounds__(256) void group_fill_kernel(const int *__restrict__ ids, int M, int K, int E,
                                                         int *__restrict__ start_out, int *__restrict__ n_slots,
                                                         int *__restrict__ slot_expert, int *__restrict__ slot_start,
                                                         int *__restrict__ slot_count, int *__restrict__ n_picks,
                                                         int *__restrict__ pick_token, int *__restrict__ pick_of) {
    __shared__ int cnt[257];
    __shared__ int wt[kFillBatch][4];
    __shared__ int part[2][4];
    const int e = static_cast<int>(blockIdx.x), tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i <= E; i += blockDim.x) cnt[i] = i == E ? M : 0;
    __syncthreads();
    for (int c0 = 0; c0 < M * K; c0 += kFillBatch * 256) {   // kFillBatch ids a thread loaded at once, then counted
        int idv[kFillBatch];
#pragma unroll
        for (int u = 0; u < kFillBatch; ++u) idv[u] = ids[min(c0 + u * 256 + tid, M * K - 1)];
#pragma unroll
        for (int u = 0; u < kFillBatch; ++u)
            if (c0 + u * 256 + tid < M * K) atomicAdd(&cnt[idv[u]], 1);
    }
    __syncthreads();
    int c = 0, s = 0;
    for (int i = tid; i < e; i += blockDim.x) {
        const int n = cnt[i];
        c += n;
        s += (n + 31) / 32;
    }
    c = wave_sum_xor(c, 64);
    s = wave_sum_xor(s, 64);
    if (lane == 0) part[0][wave] = c, part[1][wave] = s;
    __syncthreads();
    const int start = part[0][0] + part[0][1] + part[0][2] + part[0][3];
    const int sbase = part[1][0] + part[1][1] + part[1][2] + part[1][3];
    const int ce = cnt[e];
    if (tid == 0) {
        start_out[e] = start;
        if (e == E) *n_slots = sbase + (ce + 31) / 32, *n_picks = start + ce;
    }
    for (int j = tid; 32 * j < ce; j += blockDim.x) {
        slot_expert[sbase + j] = e;
        slot_start[sbase + j] = start + 32 * j;
        slot_count[sbase + j] = min(32, ce - 32 * j);
    }
    fill_expert_picks(ids, M, K, E, e, start, pick_token, pick_of, wt);
}

}  // namespace

GV_ACT_MODE_SETTER(act_mode_set_prefill)

int prefill_front(const uint16_t *gate_row, int H, const float *h, int M, int E, int K, float *logits, _Float16 *act,
                  int64_t act_stride, int *ids, float *w, float *gate, hipStream_t st) {
    GV_REQUIRE(M > 0 && H % 16 == 0 && H <= kPrefillFrontMaxH && E >= 1 && E + 1 <= 257 && K >= 1 && K <= 16 && K <= E,
               "prefill front: M > 0, hidden a multiple of 16 up to 4096, 1 <= top_k <= 16, top_k <= experts <= 256");
    const int g = (M + 3) / 4;
    const size_t lds = std::max(static_cast<size_t>(5) * H * 4, static_cast<size_t>(4) * (E + 4) * 4);
    static int granted = 0;
    if (lds_grant(reinterpret_cast<const void *>(&prefill_front_kernel), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(prefill_front_kernel, dim3(static_cast<unsigned>(2 * g + M)), dim3(256), lds, st, gate_row, H,
                       h, M, E, K, logits, act, act_stride, ids, w, gate);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int prefill_group(const int *ids, int M, int K, int E, int *start, int *n_slots, int *slot_expert, int *slot_start,
                  int *slot_count, int *n_picks, int *pick_token, int *pick_of, hipStream_t st) {
    GV_REQUIRE(M > 0 && E >= 1 && E + 1 <= 257 && K >= 1 && K <= 16, "prefill group: 1 <= top_k <= 16, experts <= 256");
    hipLaunchKernelGGL(group_fill_kernel, dim3(static_cast<unsigned>(E + 1)), dim3(256), 0, st, ids, M, K, E, start,
                       n_slots, slot_expert, slot_start, slot_count, n_picks, pick_token, pick_of);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace gv
