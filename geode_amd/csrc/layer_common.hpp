// layer_common.hpp - device code of the verify step's layers (model.hip): the KV cache layout, the route of the
// step's rows.
#pragma once

#include "mfma_gemv.hpp"
#include "model.hpp"

namespace gv {

// The device KV cache of one layer: K [nkv][slots][hd] and V [nkv][slots / 64][hd][64] in fp16 (V transposed in
// blocks of kAttnBlock positions, so that the MFMA operands of both products are contiguous loads), or the same in
// int8 followed by the scales K [nkv][slots], V [nkv][slots] (kv_scale_index).
__device__ __host__ inline int64_t kv_scale_index(int64_t slots, int nkv, int which, int kh, int64_t slot) {
    return (static_cast<int64_t>(which) * nkv + kh) * slots + slot;
}
__device__ __host__ inline int64_t k_index(int64_t slots, int hd, int kh, int64_t slot, int d) {
    return (static_cast<int64_t>(kh) * slots + slot) * hd + d;
}
__device__ __host__ inline int64_t v_index(int64_t slots, int hd, int nkv, int kh, int64_t slot, int d) {
    return static_cast<int64_t>(nkv) * slots * hd +
           ((static_cast<int64_t>(kh) * (slots / kAttnBlock) + slot / kAttnBlock) * hd + d) * kAttnBlock + slot % kAttnBlock;
}

// Row r of a tile-layout q4 matrix dequantized as dequant_row does (pack.cpp:356-366; level x E4M3 x global, bit for
// bit) into the registers norm_quant_regs takes (thread i: the 8-value groups i, i + blockDim, ..., zeros past the
// row), and to out (fp32, may be null). cols at most 32 x blockDim.
__device__ inline void dequant_row_regs(const Q4 &w, int64_t r, float (&v)[4][8], float *out) {
    const int ng = static_cast<int>(w.cols / 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int g = threadIdx.x + q * blockDim.x;   // the row's code word g (tile layout)
#pragma unroll
        for (int b = 0; b < 8; ++b) v[q][b] = 0.0f;
        if (g >= ng) continue;
        uint32_t word, sb;
        tq4_word(w, r, g, word, sb);
        const float s = __fmul_rn(e4m3_to_f32(sb), w.global);
#pragma unroll
        for (int b = 0; b < 8; ++b)
            v[q][b] = __fmul_rn(static_cast<float>(2 * static_cast<int>((word >> (4 * b)) & 15u) - 15), s);
        if (out) {
            *reinterpret_cast<float4 *>(out + g * 8) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
            *reinterpret_cast<float4 *>(out + g * 8 + 4) = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
        }
    }
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

__host__ __device__ inline int attn_k_ld(int hd) { return hd + 8; }   // halves a staged key row (bank spread)
constexpr int kAttnVld = kAttnBlock + 8;                              // halves a staged value row
inline size_t attn_lds(int hd) { return (static_cast<size_t>(kAttnBlock) * attn_k_ld(hd) + hd * kAttnVld) * 2; }

// route_topk (model.cpp:4021-4065) of NR rows by one wave, the rows' dependency chains interleaved: softmax over the
// E <= 256 experts (max, expf, the sum, divide), the top K by probability with ties to the lower index, the weights
// p / (their sum in rank order) to w[r][0..K), the ids to ids[r][0..K) (lane 0), the shared expert's gate
// sigmoid(lg[E]) to gate[r]. Lane l holds experts 4 l .. 4 l + 3, so a pick is a wave max of the lanes' largest, one
// ballot (the lowest lane holding it) and that lane's first slot holding it: the lowest index. The softmax
// denominator is a fixed tree (each lane's four values, then the lanes: wave_sum_f), not the reference's index-order
// loop: the probabilities differ from it by an ulp or so, their order (the picks) not at all. live[r] false: row r
// is skipped (its outputs untouched).
template <int NR>
__device__ inline void route_rows(const float *const (&lg)[NR], const bool (&live)[NR], int E, int K,
                                  int *const (&ids)[NR], float *const (&w)[NR], float *const (&gate)[NR],
                                  bool keep = true) {
    const int lane = threadIdx.x & 63;
    float pv[NR][4], sum[NR], raw[NR][4], lge[NR];
    // every logit up front (indices clamped, no branch around a load), the shared expert's gate logit too
#pragma unroll
    for (int r = 0; r < NR; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[r][i] = lg[r][min(4 * lane + i, E - 1)];
        lge[r] = lg[r][E];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float v[4];
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            v[i] = live[r] && e < E ? raw[r][i] : -__builtin_inff();
            mx = fmaxf(mx, v[i]);
        }
        if (r == 0) trace(GV_K_ROUTE, 5);
        mx = wave_max_all_f(mx);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            pv[r][i] = live[r] && e < E ? expf(__fsub_rn(v[i], mx)) : 0.0f;
        }
        sum[r] = wave_sum_f(__fadd_rn(__fadd_rn(pv[r][0], pv[r][1]), __fadd_rn(pv[r][2], pv[r][3])));
    }
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            pv[r][i] = live[r] && e < E ? __fdiv_rn(pv[r][i], sum[r]) : -1.0f;
        }
    trace(GV_K_ROUTE, 6);
    float top[NR], mine[NR];
    int key[NR][4];   // the probabilities' bits (non-negative: ordered as ints); taken and past E: -1.0f's (negative)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        top[r] = mine[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) key[r][i] = __float_as_int(pv[r][i]);
    }
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int lm = max(max(key[r][0], key[r][1]), max(key[r][2], key[r][3]));
            const int bk = wave_max_all_i(lm);
            const float bv = __int_as_float(bk);
            // the lowest index holding it: the lowest lane (a valid probability is >= 0 > the taken keys, so some
            // lane holds it), then that lane's first slot
            const int L = __builtin_ctzll(__ballot(lm == bk));
            const int li = key[r][0] == bk ? 0 : key[r][1] == bk ? 1 : key[r][2] == bk ? 2 : 3;
            const int bi = 4 * L + __builtin_amdgcn_readlane(li, L);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (lane == L && li == i) key[r][i] = __float_as_int(-1.0f);   // taken
            if (lane == k) mine[r] = bv;
            if (lane == 0 && live[r]) ids[r][k] = bi;
            top[r] = __fadd_rn(top[r], bv);   // rank order
        }
    }
    trace(GV_K_ROUTE, 7);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (!live[r] || !keep) continue;   // (keep false: the ids alone)
        if (lane < K) w[r][lane] = __fdiv_rn(mine[r], top[r]);
        if (lane == 0) *gate[r] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-lge[r])));
    }
}

// one row (route_rows of a single row)
__device__ inline void route_row(const float *__restrict__ lg, int E, int K, int *ids, float *w, float *gate) {
    const float *const l1[1] = {lg};
    const bool live[1] = {true};
    int *const i1[1] = {ids};
    float *const w1[1] = {w};
    float *const g1[1] = {gate};
    route_rows<1>(l1, live, E, K, i1, w1, g1);
}

// The route of the step's rows (route_rows, two rows a wave); then the slots and their picks ordered by (expert,
// token, rank), each pick placed by counting (the rows before it that picked the same expert: a bit mask per expert),
// so the order never depends on timing. A slot is a run of at most kSlotRows picks of one expert: the distinct
// experts ascending, the shared one last (index E), an expert with more picks taking consecutive slots. The whole workgroup
// (blockDim a multiple of 64, at least 256) calls this; LDS: ids [M][16], cnt / start / slot_of / rows [E + 1],
// wtot [2][16].
struct RouteLds {
    int *ids, *cnt, *start, *slot_of;
    unsigned *rows;
    int (*wtot)[16];
};

// The route's part every caller shares (the whole workgroup calls it): the rows' top-K into r.ids (route_rows; the
// weights and the shared gate to weight [M][K] / gate [M] when not null), each expert's pick count and row mask, then
// the exclusive scans: r.start[e] (its first pick), r.slot_of[e] (its first slot, -1: none), and the slot and pick
// totals in r.wtot[0][15] / r.wtot[1][15]. Every result is the same whatever the timing (counts, masks and scans).
__device__ inline void route_core(const float *__restrict__ logits, int E, int K, int M, float *weight, float *gate,
                                  const RouteLds &r) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, waves = blockDim.x >> 6;
    const int E1 = E + 1;
    trace(GV_K_ROUTE, 0);
    for (int e = tid; e <= E; e += blockDim.x) r.cnt[e] = 0, r.rows[e] = 0;
    // (no weight: route_rows writes the ids alone, never w or g)
    if (M < 2 * waves) {   // a row a wave (the first M - waves waves a second one after it: a pair in every wave
                           // would run the second row's instructions, masked, in all of them)
        for (int t0 = wave; t0 < M; t0 += waves) {
            const float *const lg[1] = {logits + static_cast<int64_t>(t0) * E1};
            const bool live[1] = {true};
            int *const ids[1] = {&r.ids[t0 * 16]};
            float *const w[1] = {weight ? weight + t0 * K : nullptr};
            float *const g[1] = {gate ? gate + t0 : nullptr};
            route_rows<1>(lg, live, E, K, ids, w, g, weight != nullptr);
        }
    } else {
        for (int t0 = wave; t0 < M; t0 += 2 * waves) {   // rows t0 and t0 + waves
            const int t1 = t0 + waves;
            const bool l1 = t1 < M;
            const int t1c = l1 ? t1 : t0;
            const float *const lg[2] = {logits + static_cast<int64_t>(t0) * E1,
                                        logits + static_cast<int64_t>(t1c) * E1};
            const bool live[2] = {true, l1};
            int *const ids[2] = {&r.ids[t0 * 16], &r.ids[t1c * 16]};
            float *const w[2] = {weight ? weight + t0 * K : nullptr, weight ? weight + t1c * K : nullptr};
            float *const g[2] = {gate ? gate + t0 : nullptr, gate ? gate + t1c : nullptr};
            route_rows<2>(lg, live, E, K, ids, w, g, weight != nullptr);
        }
    }
    __syncthreads();
    trace(GV_K_ROUTE, 1);
    for (int i = tid; i < M * K; i += blockDim.x) {
        const int t = i / K, e = r.ids[t * 16 + i % K];
        atomicAdd(&r.cnt[e], 1);
        atomicOr(&r.rows[e], 1u << t);
    }
    if (tid == 0) r.cnt[E] = M;
    __syncthreads();
    trace(GV_K_ROUTE, 2);
    {   // exclusive scans over the E + 1 counters (starts, slot numbers): two a thread, waves, the waves' totals
        const int e0 = 2 * tid, e1 = e0 + 1;
        const int c0 = e0 <= E ? r.cnt[e0] : 0, c1 = e1 <= E ? r.cnt[e1] : 0;
        const int u0 = (c0 + kSlotRows - 1) / kSlotRows, u1 = (c1 + kSlotRows - 1) / kSlotRows;   // slots
        const int ic = wave_incl_scan(c0 + c1), iu = wave_incl_scan(u0 + u1);
        if (lane == 63) r.wtot[0][wave] = ic, r.wtot[1][wave] = iu;
        __syncthreads();
        int bc = 0, bu = 0;
        for (int w2 = 0; w2 < wave; ++w2) bc += r.wtot[0][w2], bu += r.wtot[1][w2];
        const int xc = bc + ic - (c0 + c1), xu = bu + iu - (u0 + u1);   // exclusive, before e0
        if (e0 <= E) {
            r.start[e0] = xc;
            r.slot_of[e0] = u0 ? xu : -1;   // the expert's first slot
        }
        if (e1 <= E) {
            r.start[e1] = xc + c0;
            r.slot_of[e1] = u1 ? xu + u0 : -1;
        }
        __syncthreads();   // (every wave has read the totals)
        if (e0 == E || e1 == E) {   // the totals, for the callers
            r.wtot[1][15] = xu + u0 + (e1 == E ? u1 : 0);
            r.wtot[0][15] = xc + c0 + (e1 == E ? c1 : 0);
        }
    }
    __syncthreads();
    trace(GV_K_ROUTE, 3);
}

// The slot tables of the route in LDS (route_core's) written to the route state, with the ids (route_all's tail)
__device__ inline void route_tables(int E, int K, int M, RouteState *__restrict__ rs, int32_t *__restrict__ ids_out,
                                    const RouteLds &r) {
    const int tid = threadIdx.x;
    if (tid == 0) rs->n_slots = r.wtot[1][15], rs->n_picks = r.wtot[0][15];
    for (int i = tid; i < M * K; i += blockDim.x) ids_out[i] = r.ids[(i / K) * 16 + i % K];
    for (int e = tid; e <= E; e += blockDim.x)
        if (r.slot_of[e] >= 0)
            for (int k = 0; k * kSlotRows < r.cnt[e]; ++k) {
                const int u = r.slot_of[e] + k;
                rs->slot_expert[u] = e;
                rs->slot_start[u] = r.start[e] + k * kSlotRows;
                rs->slot_count[u] = min(kSlotRows, r.cnt[e] - k * kSlotRows);
            }
    // pick (t, k) of expert e goes after the earlier rows' picks of e (a row picks an expert at most once); its
    // row also goes to its slot's token list (a slot's unused entries: the slot's first row, by the pick before = 0
    // of each slot writing them)
    for (int i = tid; i < M * (K + 1); i += blockDim.x) {
        const int t = i / (K + 1), k = i % (K + 1);
        const int e = k < K ? r.ids[t * 16 + k] : E;
        const int before = k < K ? __popc(r.rows[e] & ((1u << t) - 1u)) : t;
        const int pk = r.start[e] + before;
        rs->pick_token[pk] = t;
        rs->pick_of[t * (K + 1) + k] = pk;
        const int u = r.slot_of[e] + before / kSlotRows, j = before % kSlotRows;
        const int n = min(kSlotRows, r.cnt[e] - (before / kSlotRows) * kSlotRows);
        rs->slot_dst[u * kSlotRows + j] = t * (K + 1) + k;
        if (j > 0) {
            rs->slot_token[u * kSlotRows + j] = t;
        } else {
            for (int jj = n; jj < kSlotRows; ++jj) rs->slot_token[u * kSlotRows + jj] = t;
            rs->slot_token[u * kSlotRows] = t;
        }
    }
    trace(GV_K_ROUTE, 4);
}

// The route of the step's rows (route_rows, two rows a wave); then the slots and their picks ordered by (expert,
// token, rank), each pick placed by counting (the rows before it that picked the same expert: a bit mask per expert),
// so the order never depends on timing. A slot is a run of at most kSlotRows picks of one expert: the distinct
// experts ascending, the shared one last (index E), an expert with more picks taking consecutive slots. The whole
// workgroup (blockDim a multiple of 64, at least 256) calls this; LDS: ids [M][16], cnt / start / slot_of / rows
// [E + 1], wtot [2][16].
__device__ inline void route_all(const float *__restrict__ logits, int E, int K, int M, RouteState *__restrict__ rs,
                                 int32_t *__restrict__ ids_out, const RouteLds &r) {
    route_core(logits, E, K, M, rs->weight, rs->gate, r);
    route_tables(E, K, M, rs, ids_out, r);
}

// The route of at most 8 rows of at most 8 picks (M K <= 64, E <= 256) for one workgroup of the experts' up launch:
// route_core's results in LDS (the same ids, counts, row masks, starts and slot numbers: its top-K branch, then the
// counts and both scans by one wave, an expert's count being at most M <= kSlotRows so one slot at most), and slot
// u's expert, first pick, pick count and row mask in sel[0..3] (sel[0] = -1: u is past the slots). Two barriers.
__device__ inline void route_small(const float *__restrict__ logits, int E, int K, int M, float *weight, float *gate,
                                   const RouteLds &r, int u, int *sel) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, waves = blockDim.x >> 6;
    const int E1 = E + 1;
    trace(GV_K_ROUTE, 0);
    for (int e = tid; e <= E; e += blockDim.x) r.cnt[e] = 0, r.rows[e] = 0;
    // (no weight: route_rows writes the ids alone, never w or g)
    if (M < 2 * waves) {   // (route_core's branches: the same rows on the same arithmetic)
        for (int t0 = wave; t0 < M; t0 += waves) {
            const float *const lg[1] = {logits + static_cast<int64_t>(t0) * E1};
            const bool live[1] = {true};
            int *const ids[1] = {&r.ids[t0 * 16]};
            float *const w[1] = {weight ? weight + t0 * K : nullptr};
            float *const g[1] = {gate ? gate + t0 : nullptr};
            route_rows<1>(lg, live, E, K, ids, w, g, weight != nullptr);
        }
    } else {
        for (int t0 = wave; t0 < M; t0 += 2 * waves) {
            const int t1 = t0 + waves;
            const bool l1 = t1 < M;
            const int t1c = l1 ? t1 : t0;
            const float *const lg[2] = {logits + static_cast<int64_t>(t0) * E1,
                                        logits + static_cast<int64_t>(t1c) * E1};
            const bool live[2] = {true, l1};
            int *const ids[2] = {&r.ids[t0 * 16], &r.ids[t1c * 16]};
            float *const w[2] = {weight ? weight + t0 * K : nullptr, weight ? weight + t1c * K : nullptr};
            float *const g[2] = {gate ? gate + t0 : nullptr, gate ? gate + t1c : nullptr};
            route_rows<2>(lg, live, E, K, ids, w, g, weight != nullptr);
        }
    }
    __syncthreads();
    trace(GV_K_ROUTE, 1);
    if (wave == 0) {
        const int np = M * K;
        if (lane < np) {   // (one wave's LDS operations complete in order: the reads below see every count)
            const int t = lane / K, e = r.ids[t * 16 + lane % K];
            atomicAdd(&r.cnt[e], 1);
            atomicOr(&r.rows[e], 1u << t);
        }
        int c[4], n = 0, s = 0;   // experts 4 lane .. 4 lane + 3: their picks and slots
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            c[j] = e < E ? r.cnt[e] : 0;
            n += c[j];
            s += c[j] > 0 ? 1 : 0;
        }
        const int is = wave_incl_scan(s), in = wave_incl_scan(n);
        const int U = __builtin_amdgcn_readlane(is, 63);   // the routed experts' slots (the shared one's is U)
        int sl = is - s, st = in - n;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            if (e < E) {
                r.start[e] = st;
                r.slot_of[e] = c[j] ? sl : -1;
                if (c[j] && sl == u) sel[0] = e, sel[1] = st, sel[2] = c[j], sel[3] = static_cast<int>(r.rows[e]);
            }
            st += c[j];
            sl += c[j] > 0 ? 1 : 0;
        }
        if (lane == 0) {
            r.cnt[E] = M;
            r.start[E] = np;
            r.slot_of[E] = U;
            r.wtot[0][15] = np + M;   // (the totals, as route_core leaves them)
            r.wtot[1][15] = U + 1;
            if (u == U) sel[0] = E, sel[1] = np, sel[2] = M, sel[3] = static_cast<int>((1u << M) - 1u);
            else if (u > U) sel[0] = -1;
        }
    }
    __syncthreads();
    trace(GV_K_ROUTE, 3);
}

// The post-attention RMSNorm (none when norm_w is null: the rows are used as they are) and the router logits. A
// workgroup takes 4 rows of the router ([E + 1][H] bf16, the
// shared expert's gate row last; one a wave) and the tokens in groups of router_tokens(H). Every load is issued
// first (the rows, the residual rows, the norm weights); the sums of squares, 1 / RMS and x inv (1 + w) (rmsnorm's
// arithmetic) then come from registers, workgroup b also writing token b's operands for the experts' products, and
// the normalized rows and the router rows (as fp32) go to LDS for the sums. Each logit is eight partial sums in the
// reference's fixed order (bf16_row_dots, kernels.cpp:1446-1483), a lane per (token, partial).
constexpr int kRouterRows = 4;
__host__ __device__ inline int router_tokens(int H) { return H <= 2048 ? 8 : 4; }
// the route's LDS in the router's tail: p [kMaxRows][256], ids [kMaxRows][16], cnt / start / slot_of [257]
constexpr size_t kRouteLds = (static_cast<size_t>(kMaxRows) * 16 + 4 * 260) * 4;
inline size_t router_lds(int H) {
    return std::max(static_cast<size_t>(router_tokens(H)) * (H + 8) * 4 + static_cast<size_t>(kRouterRows) * H * 4,
                    kRouteLds);
}


// The router's rows for workgroup (wg, token groups tg0, tg0 + tg_step, ..) (router_kernel's body; also the a / b dots
// of a Gated DeltaNet layer, gdn.hip): logits [M][E1] of the rows (RMSNorm(x) with norm_w, or x as it is when null) of
// those groups of router_tokens(H) rows against bf16 rows [wg 4, wg 4 + 4) of w; out_sc1: the logits stored with the
// sc1 policy (read later in the same launch); act (not null) and act_row >= 0: the workgroup also writes row act_row's
// operands for the experts' products (a row of its groups).
template <int GPT>   // 8-value groups a thread takes per row: 1 for H <= 2048, 2 up to 4096
__device__ inline void router_rows(int wg, int tg0, int tg_step, const uint16_t *__restrict__ w, int E1, int H,
                                   const float *__restrict__ x, const float *__restrict__ norm_w, float eps,
                                   const StepParams *__restrict__ sp, float *__restrict__ logits, bool out_sc1,
                                   _Float16 *__restrict__ act, int act_row, int64_t act_stride, float *lds_f) {
    constexpr int TG = GPT == 1 ? 8 : 4;
    __shared__ double red[4][TG];
    const int ldh = H + 8;
    float *hs = lds_f;                 // [TG][ldh] the normalized rows
    float *ws = hs + TG * ldh;         // [4][H] the router rows as fp32
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    trace(GV_K_ROUTER, 0);
    const int M = sp->M, r0 = wg * kRouterRows;
    // Every load is unconditional (indices clamped into the arrays), so that none waits for the ones before it:
    // the first group's rows (needed first), the norm weights, then the workgroup's router rows (4 x H bf16, 8 a
    // load, H / 256 loads a thread; rows past E1 read row E1 - 1 and are never used).
    float xv[TG][GPT][8];
    const float *zero = reinterpret_cast<const float *>(g_zero_act16);   // 64 KB of zeros
    auto load_x = [&](int t0) {   // (rows past the group's count: a copy of its last, unused; columns past H: 0)
        const int nt = min(TG, M - t0);
#pragma unroll
        for (int tt = 0; tt < TG; ++tt)
#pragma unroll
            for (int q = 0; q < GPT; ++q) {
                const int g = threadIdx.x + q * 256;
                const float *src = g < H / 8 ? x + static_cast<int64_t>(t0 + min(tt, nt - 1)) * H + g * 8 : zero;
                const float4 a = *reinterpret_cast<const float4 *>(src), b = *reinterpret_cast<const float4 *>(src + 4);
                const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[tt][q][i] = t[i];
            }
    };
    const int first = tg0 * TG;
    if (first >= M) return;   // (uniform: no rows for this workgroup)
    load_x(first);
    float nw[GPT][8];   // 1 + w (no norm: w read from the zeros)
#pragma unroll
    for (int q = 0; q < GPT; ++q) {
        const int g = threadIdx.x + q * 256;
        const float *src = norm_w && g < H / 8 ? norm_w + g * 8 : zero;
        const float4 a = *reinterpret_cast<const float4 *>(src), b = *reinterpret_cast<const float4 *>(src + 4);
        const float t[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) nw[q][i] = __fadd_rn(1.0f, t[i]);
    }
    uint4 wr[GPT * 4];
#pragma unroll
    for (int k = 0; k < GPT * 4; ++k) {
        const int i = min(static_cast<int>(threadIdx.x) + k * 256, 4 * (H / 8) - 1), rr = i / (H / 8), c8 = i % (H / 8);
        wr[k] = *reinterpret_cast<const uint4 *>(w + static_cast<int64_t>(min(r0 + rr, E1 - 1)) * H + c8 * 8);
    }
    // one group of up to TG rows: 1 / RMS per row (the thread's squares, the wave sums, the waves' in order), the
    // normalized rows to LDS (and row wg's operands), then the dots
    auto group = [&](int t0, bool first) {
        const int nt = min(TG, M - t0);
        if (!first) __syncthreads();   // the previous group's dots are done with hs and red
        trace(GV_K_ROUTER, 1);
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) {
            if (tt >= nt) break;   // uniform
            double ss = 0.0;
#pragma unroll
            for (int q = 0; q < GPT; ++q)
#pragma unroll
                for (int i = 0; i < 8; ++i) ss += static_cast<double>(xv[tt][q][i]) * static_cast<double>(xv[tt][q][i]);
            ss = wave_sum(ss);
            if (lane == 0) red[wave][tt] = ss;
        }
        if (first) {   // the router rows to LDS as fp32
#pragma unroll
            for (int k = 0; k < GPT * 4; ++k) {
                const int i = threadIdx.x + k * 256;
                if (i >= 4 * (H / 8)) break;
                const uint32_t u[4] = {wr[k].x, wr[k].y, wr[k].z, wr[k].w};
                float *d = ws + (i / (H / 8)) * H + (i % (H / 8)) * 8;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    d[2 * h] = __uint_as_float(u[h] << 16);
                    d[2 * h + 1] = __uint_as_float(u[h] & 0xFFFF0000u);
                }
            }
        }
        __syncthreads();
        const int tq = act_row - t0;
#pragma unroll
        for (int tt = 0; tt < TG; ++tt) {
            if (tt >= nt) break;
            const double tot = ((red[0][tt] + red[1][tt]) + red[2][tt]) + red[3][tt];
            const float inv =
                norm_w ? __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(tot / static_cast<double>(H)), eps)))
                       : 1.0f;
#pragma unroll
            for (int q = 0; q < GPT; ++q) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = __fmul_rn(__fmul_rn(xv[tt][q][i], inv), nw[q][i]);
                const int g = threadIdx.x + q * 256;
                const bool live = g < H / 8;
                if (live) {
                    *reinterpret_cast<float4 *>(hs + tt * ldh + g * 8) = make_float4(v[0], v[1], v[2], v[3]);
                    *reinterpret_cast<float4 *>(hs + tt * ldh + g * 8 + 4) = make_float4(v[4], v[5], v[6], v[7]);
                }
                if (act && tt == tq) act16_group(v, g, live, act + static_cast<int64_t>(act_row) * act_stride);
            }
        }
        __syncthreads();
        trace(GV_K_ROUTER, 2);
        const int tt = lane / 8, j = lane % 8;
        const int ra = r0 + wave;
        if (ra >= E1) return;
        const float *hr = hs + (tt < nt ? tt : 0) * ldh;
        const float *wrow = ws + wave * H;
        float a0 = 0.0f;
        for (int c0 = j; c0 < H; c0 += 8 * 16) {   // 16 steps' operands read ahead of their sums
            float hv[16], wv[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                hv[u] = hr[c0 + 8 * u];
                wv[u] = wrow[c0 + 8 * u];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) a0 = __fadd_rn(a0, __fmul_rn(wv[u], hv[u]));
        }
        // ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7))
        const float s1 = __fadd_rn(a0, __shfl_down(a0, 4, 64));
        const float s2 = __fadd_rn(s1, __shfl_down(s1, 1, 64));
        const float s3 = __fadd_rn(s2, __shfl_down(s2, 2, 64));
        if (j == 0 && tt < nt) {
            const int64_t li = static_cast<int64_t>(t0 + tt) * E1 + ra;
            if (out_sc1) xstf(logits, static_cast<uint32_t>(li), s3);
            else logits[li] = s3;
        }
    };
    group(first, true);
    for (int t0 = first + tg_step * TG; t0 < M; t0 += tg_step * TG) {
        load_x(t0);
        group(t0, false);
    }
    trace(GV_K_ROUTER, 3);
}

}  // namespace gv
