// The prefill MoE's (C5) work before the experts' products, in two launches instead of five: the rows' routes, then
// the grouping of their picks by expert with the picks' placement, the shared expert's gate and the products'
// operands as roles of one launch (the gate, the slowest, beside the grouping that waits on the routes). Each output
// is what the separate kernels (model.hip: gate_rows_kernel, route_rows_kernel, quantize_act_kernel, group_kernel,
// fill_picks_kernel) write, bit for bit; gv_model_set_fused(m, 0) runs those instead. The kernels live in this source
// file of their own so that the verify step's kernels keep their places in model.hip's code object.
#include <algorithm>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"
#include "prefill_common.hpp"

namespace gv {
namespace {

// the rows' top K and their weights (route_row), 4 rows a workgroup of 256 threads, on a copy of each row's E routed
// logits in LDS (column E, the shared expert's gate logit, is not read: the gate role makes the gate itself;
// route_row's gate output goes to that LDS slot, unused)
__global__ __launch_bounds__(256) void prefill_route_kernel(const float *__restrict__ logits, int M, int E, int K,
                                                            int *__restrict__ ids, float *__restrict__ w) {
    __shared__ float rows[4][257 + 3];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, E1 = E + 1;
    const int t = static_cast<int>(blockIdx.x) * 4 + wave;
    if (t >= M) return;   // (no barrier below: a wave's own row)
    float *row = rows[wave];
    const float *src = logits + static_cast<int64_t>(t) * E1;
    for (int i = lane; i < E; i += 64) row[i] = src[i];
    if (lane == 0) row[E] = 0.0f;
    // (one wave's LDS operations complete in order: route_row's reads see the copy)
    route_row(row, E, K, ids + static_cast<int64_t>(t) * K, w + static_cast<int64_t>(t) * K, &row[E]);
}

// The picks of expert e grouped and placed (a workgroup of 256 threads): every expert's pick count into LDS (the
// shared expert E takes every row), e's first pick and first slot as the sums of the counts and of the slot counts
// below e (integers: any order), e's slots (runs of at most 32 picks) and its picks' places (fill_expert_picks); the
// workgroup of E also writes the totals. group_kernel and fill_picks_kernel's outputs.
struct GroupOut {
    int *start, *n_slots, *slot_expert, *slot_start, *slot_count, *n_picks, *pick_token, *pick_of;
};
__device__ void group_fill(const int *__restrict__ ids, int M, int K, int E, int e, const GroupOut &o) {
    __shared__ int cnt[257];
    __shared__ int wt[kFillBatch][4];
    __shared__ int part[2][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
        o.start[e] = start;
        if (e == E) *o.n_slots = sbase + (ce + 31) / 32, *o.n_picks = start + ce;
    }
    for (int j = tid; 32 * j < ce; j += blockDim.x) {
        o.slot_expert[sbase + j] = e;
        o.slot_start[sbase + j] = start + 32 * j;
        o.slot_count[sbase + j] = min(32, ce - 32 * j);
    }
    fill_expert_picks(ids, M, K, E, e, start, o.pick_token, o.pick_of, wt);
}

// Three roles after the routes, g = ceil(M / 4), G = E + 1 (or 0: no grouping), 256 threads:
//   workgroups [0, g)                  the shared expert's gate logits (gate_row_logit, 4 rows a workgroup) to
//                                      logits [t][E] and sigmoid(logit) to gate [t] (route_rows' arithmetic,
//                                      model.cpp:4021-4065);
//   workgroups [g, g + G)              expert b - g's picks grouped and placed (group_fill);
//   workgroups [g + G, g + G + M)      row t's operands for the products (norm_quant_row without a norm,
//                                      quantize_act's).
__global__ __launch_bounds__(256) void prefill_rest_kernel(const uint16_t *__restrict__ wrow, int H,
                                                           const float *__restrict__ h, int M, int E, int K,
                                                           float *__restrict__ logits, float *__restrict__ gate,
                                                           _Float16 *__restrict__ act, int64_t act_stride,
                                                           const int *__restrict__ ids, const GroupOut o, int G) {
    extern __shared__ float pf_lds[];
    __shared__ double red[16];
    const int g = (M + 3) / 4, b = static_cast<int>(blockIdx.x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (b < g) {
        const int t = b * 4 + wave;
        const float sg = gate_row_logit(wrow, H, h, M, t, pf_lds);
        if (t < M && lane == 0) {
            logits[static_cast<int64_t>(t) * (E + 1) + E] = sg;
            gate[t] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-sg)));
        }
    } else if (b < g + G) {
        group_fill(ids, M, K, E, b - g, o);
    } else {
        const int t = b - g - G;
        norm_quant_row(h + static_cast<int64_t>(t) * H, H, nullptr, 0.0f, act + static_cast<int64_t>(t) * act_stride,
                       nullptr, red);
    }
}

}  // namespace

GV_ACT_MODE_SETTER(act_mode_set_prefill)

static int g_rest_granted = 0;   // prefill_rest_kernel's dynamic LDS grant (both of its host entries)

int prefill_route(const float *logits, int M, int E, int K, int *ids, float *w, hipStream_t st) {
    GV_REQUIRE(M > 0 && E >= 1 && E + 1 <= 257 && K >= 1 && K <= 16 && K <= E,
               "prefill route: M > 0, 1 <= top_k <= 16, top_k <= experts <= 256");
    hipLaunchKernelGGL(prefill_route_kernel, dim3(static_cast<unsigned>((M + 3) / 4)), dim3(256), 0, st, logits, M, E,
                       K, ids, w);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int prefill_rest(const uint16_t *gate_row, int H, const float *h, int M, int E, int K, float *logits, float *gate,
                 _Float16 *act, int64_t act_stride, const int *ids, int *start, int *n_slots, int *slot_expert,
                 int *slot_start, int *slot_count, int *n_picks, int *pick_token, int *pick_of, hipStream_t st) {
    GV_REQUIRE(ids && start && n_slots && slot_expert && slot_start && slot_count && n_picks && pick_token && pick_of,
               "prefill: the grouping's arrays");
    GV_REQUIRE(M > 0 && H % 16 == 0 && H <= kPrefillFrontMaxH && E >= 1 && E + 1 <= 257 && K >= 1 && K <= 16,
               "prefill: M > 0, hidden a multiple of 16 up to 4096, 1 <= top_k <= 16, experts <= 256");
    const int g = (M + 3) / 4;
    const size_t lds = static_cast<size_t>(5) * H * 4;   // the gate role's: the gate row and 4 rows as fp32
    if (lds_grant(reinterpret_cast<const void *>(&prefill_rest_kernel), lds, g_rest_granted) != 0) return -1;
    const GroupOut o{start, n_slots, slot_expert, slot_start, slot_count, n_picks, pick_token, pick_of};
    hipLaunchKernelGGL(prefill_rest_kernel, dim3(static_cast<unsigned>(g + E + 1 + M)), dim3(256), lds, st, gate_row,
                       H, h, M, E, K, logits, gate, act, act_stride, ids, o, E + 1);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int prefill_gate_ops(const uint16_t *gate_row, int H, const float *h, int M, int E, float *logits, float *gate,
                     _Float16 *act, int64_t act_stride, hipStream_t st) {
    GV_REQUIRE(M > 0 && H % 16 == 0 && H <= kPrefillFrontMaxH && E >= 1 && E + 1 <= 257,
               "gate and operands: M > 0, hidden a multiple of 16 up to 4096, experts <= 256");
    const int g = (M + 3) / 4;
    const size_t lds = static_cast<size_t>(5) * H * 4;
    if (lds_grant(reinterpret_cast<const void *>(&prefill_rest_kernel), lds, g_rest_granted) != 0) return -1;
    hipLaunchKernelGGL(prefill_rest_kernel, dim3(static_cast<unsigned>(g + M)), dim3(256), lds, st, gate_row, H, h, M,
                       E, 0, logits, gate, act, act_stride, static_cast<const int *>(nullptr), GroupOut{}, 0);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

}  // namespace gv
