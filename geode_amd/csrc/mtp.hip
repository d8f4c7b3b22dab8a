// mtp.hip - the MTP draft layer on the GPU: Model::draft / draft_next (engine/src/model.cpp:1286-1479) over
// Model::forward_mtp (:4965-5039), with the draft head of draft_vocab.bin (:803-827).
//
// A pass of n rows at MTP positions pos..: row t pairs a hidden row (the verify's final-normed row, the caller's, or
// the last pass's mtp.norm output) with the token after it. The input kernel makes fc's operands from
// [RMSNorm(embedding; 1 + pre_e) | RMSNorm(hidden; 1 + pre_h)]; fc is one skinny product; the MTP layer's in-norm
// goes to the layer's operands; the decoder layer is the verify step's own launches on layer index n_layers (its KV
// cache after the main layers', its experts resident like theirs) with mtp.norm in place of the next layer's norm;
// then lm_head (or the draft head) over the last row only and the pick: the first maximum and its softmax probability
// summed in double, in two launches over 64 chunks of the logits. Everything but the result's 8 bytes stays on the
// device.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "layer_common.hpp"
#include "mfma_gemv.hpp"
#include "model.hpp"

namespace gv {

namespace {

constexpr int kPickWgs = 64;       // chunks of the logits the pick splits over
constexpr int kPickThreads = 512;

// the pick's exchange area (device): per chunk its maximum, first index and sum; the result
struct PickArea {
    float chunk_max[kPickWgs];
    int chunk_idx[kPickWgs];
    float chunk_sum[2 * kPickWgs];   // a double's two halves per chunk
    float maxv;
    int best;
    int count;   // finished workgroups of the running pick launch (zero between launches)
    int draft;
    float prob;
};

// ---------------------------------------------------------------- kernels
// fc's operands of row t (forward_mtp, model.cpp:4992-5008): the embedding of tokens[t] (dequant_row) normalized with
// 1 + pre_e in values [0, H), the hidden row hrow[t] of hbuf normalized with 1 + pre_h in [H, 2 H), each as the int8
// path's 16-value blocks (quantize_activation on the 2 H row: its blocks lie within one half, H being a multiple of
// 16). A workgroup a row.
__global__ __launch_bounds__(256) void mtp_in_kernel(Q4 emb, const StepParams *__restrict__ sp,
                                                     const float *__restrict__ hbuf, const float *__restrict__ pre_e,
                                                     const float *__restrict__ pre_h, float eps,
                                                     _Float16 *__restrict__ act, int64_t act_stride) {
    __shared__ double red[16];
    const int t = blockIdx.x;
    if (t >= sp->M) return;
    const int H = static_cast<int>(emb.cols);
    float v[4][8];
    dequant_row_regs(emb, sp->tokens[t], v, nullptr);
    _Float16 *ar = act + static_cast<int64_t>(t) * act_stride;
    norm_quant_regs(v, H, pre_e, eps, ar, nullptr, red);
    norm_quant_row(hbuf + static_cast<int64_t>(sp->hrow[t]) * H, H, pre_h, eps, ar + act_halves(H), nullptr, red);
}

// (value, index) pairs: the larger value, on equal values the lower index (std::max_element's first maximum)
__device__ inline void better(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) v = v2, i = i2;
}
__device__ inline void wave_best(float &v, int &i) {
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(v, off, 64);
        const int i2 = __shfl_xor(i, off, 64);
        better(v, i, v2, i2);
    }
}
__device__ inline int pick_chunk(int rows) { return (rows + kPickWgs - 1) / kPickWgs; }

// The maximum: per chunk its largest logit and first index (sc1 stores), then the last workgroup to finish takes the
// chunks in order (a later chunk only with a larger value: the first maximum) into maxv / best.
__global__ __launch_bounds__(kPickThreads) void pick_max_kernel(const float *__restrict__ lg, int rows, PickArea *pa) {
    __shared__ float sv[kPickThreads / 64];
    __shared__ int si[kPickThreads / 64];
    __shared__ int last;
    const int b = blockIdx.x, chunk = pick_chunk(rows);
    const int lo = b * chunk, hi = min(rows, lo + chunk);
    float v = -INFINITY;
    int idx = INT32_MAX;
    for (int i = lo + static_cast<int>(threadIdx.x); i < hi; i += kPickThreads) better(v, idx, lg[i], i);
    wave_best(v, idx);
    if (threadIdx.x % 64 == 0) sv[threadIdx.x / 64] = v, si[threadIdx.x / 64] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kPickThreads / 64; ++w) better(v, idx, sv[w], si[w]);
        xstf(pa->chunk_max, b, v);
        xstf(reinterpret_cast<float *>(pa->chunk_idx), b, __builtin_bit_cast(float, idx));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        last = __hip_atomic_fetch_add(&pa->count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kPickWgs - 1;
    }
    __syncthreads();
    if (!last || threadIdx.x != 0) return;
    float mv = -INFINITY;
    int mi = INT32_MAX;
    for (int c = 0; c < kPickWgs; ++c) {
        const float cv = xldf(pa->chunk_max, c);
        const int ci = __builtin_bit_cast(int, xldf(reinterpret_cast<const float *>(pa->chunk_idx), c));
        if (cv > mv) mv = cv, mi = ci;   // (an empty chunk: -inf, never taken)
    }
    pa->maxv = mv;
    pa->best = mi >= 0 && mi < rows ? mi : 0;   // (no maximum only when every logit is NaN)
    __hip_atomic_store(&pa->count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The probability: per chunk sum exp(double(l - max)) (the difference in fp32 as the reference's, softmax_at), then the
// last workgroup adds the chunks' sums in order: prob = 1 / sum, draft = the best index (through ids when a draft
// vocabulary is set).
__global__ __launch_bounds__(kPickThreads) void pick_sum_kernel(const float *__restrict__ lg, int rows,
                                                                const int32_t *__restrict__ ids, PickArea *pa) {
    __shared__ double sd[kPickThreads / 64];
    __shared__ int last;
    const int b = blockIdx.x, chunk = pick_chunk(rows);
    const int lo = b * chunk, hi = min(rows, lo + chunk);
    const float mv = pa->maxv;
    double s = 0.0;
    for (int i = lo + static_cast<int>(threadIdx.x); i < hi; i += kPickThreads)
        s += exp(static_cast<double>(__fsub_rn(lg[i], mv)));
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (threadIdx.x % 64 == 0) sd[threadIdx.x / 64] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = 0.0;
        for (int w = 0; w < kPickThreads / 64; ++w) tot += sd[w];
        const uint64_t bits = __builtin_bit_cast(uint64_t, tot);
        xstf(pa->chunk_sum, 2 * b, __builtin_bit_cast(float, static_cast<uint32_t>(bits)));
        xstf(pa->chunk_sum, 2 * b + 1, __builtin_bit_cast(float, static_cast<uint32_t>(bits >> 32)));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        last = __hip_atomic_fetch_add(&pa->count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kPickWgs - 1;
    }
    __syncthreads();
    if (!last || threadIdx.x != 0) return;
    double tot = 0.0;
    for (int c = 0; c < kPickWgs; ++c) {
        const uint64_t lo32 = __builtin_bit_cast(uint32_t, xldf(pa->chunk_sum, 2 * c));
        const uint64_t hi32 = __builtin_bit_cast(uint32_t, xldf(pa->chunk_sum, 2 * c + 1));
        tot += __builtin_bit_cast(double, lo32 | (hi32 << 32));
    }
    pa->prob = static_cast<float>(1.0 / tot);
    pa->draft = ids ? ids[pa->best] : pa->best;
    __hip_atomic_store(&pa->count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row i of the draft head = row ids[i] of lm_head, tile layout to tile layout: a code word's place in its tile and its
// scale byte's depend on the row within the tile only, so both move as they are. A thread a (row, code word).
__global__ void draft_rows_kernel(Q4 src, const int32_t *__restrict__ ids, int n, uint8_t *__restrict__ codes,
                                  uint8_t *__restrict__ scales) {
    const int64_t nw = src.cols / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(n) * nw) return;
    const int64_t r = i / nw, wi = i % nw, sr = ids[r];
    const int64_t nsc = src.cols / kSuperK, nsq = (nsc + 3) / 4, sc = wi / 16, j = (wi % 16) / 4, g = wi % 4;
    const int64_t T = r / kTileR, rr = r % kTileR, ST = sr / kTileR, srr = sr % kTileR;
    *reinterpret_cast<uint32_t *>(codes + (T * nsc + sc) * 1024 + (rr + 16 * g) * 16 + j * 4) =
        *reinterpret_cast<const uint32_t *>(src.codes + (ST * nsc + sc) * 1024 + (srr + 16 * g) * 16 + j * 4);
    if (g % 2 == 0) scales[tq4_scale_off(T, nsq, sc, rr, g, j)] = src.scales[tq4_scale_off(ST, nsq, sc, srr, g, j)];
}

// ---------------------------------------------------------------- host side
void *mtp_dalloc(Model &m, size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
    m.allocs.push_back(p);
    return p;
}

int64_t head_rows(const Model &m) { return m.draft_head.rows > 0 ? m.draft_head.rows : m.c.vocab; }

// The pass's parameters: n rows at pos, their tokens and hidden rows (hbuf rows), a chain
int mtp_params(Model &m, const int32_t *toks, int n, int pos, const int *hrow, const char *who) {
    const auto &c = m.c;
    GV_REQUIRE(m.has_mtp, std::string(who) + ": the model has no MTP layer");
    GV_REQUIRE(n >= 1 && n <= c.max_rows, std::string(who) + ": 1 <= n <= max_rows");
    GV_REQUIRE(pos >= 0 && pos + n <= c.max_ctx, std::string(who) + ": positions past the context");
    StepParams &sp = m.host_sp_mtp;
    std::memset(&sp, 0, sizeof sp);
    sp.pos = pos;
    sp.M = n;
    for (int t = 0; t < n; ++t) {
        GV_REQUIRE(toks[t] >= 0 && toks[t] < c.vocab, std::string(who) + ": token out of range");
        sp.tokens[t] = toks[t];
        sp.depth[t] = t;
        sp.vis[t] = t == 31 ? 0xFFFFFFFFu : ((1u << (t + 1)) - 1u);
        sp.hrow[t] = hrow[t];
    }
    GV_CHECK_HIP(hipMemcpyAsync(m.sp_mtp, &sp, sizeof sp, hipMemcpyHostToDevice, stream()));
    return 0;
}

// the hidden rows of a pass: the caller's (copied to the third part of hbuf) or the last verify's (the first part;
// after a keep with a path, the path's rows)
int mtp_hidden_rows(Model &m, int n, const float *hidden, int *hrow, const char *who) {
    const auto &c = m.c;
    const int H = c.hidden, Mx = c.max_rows;
    if (hidden) {
        GV_CHECK_HIP(hipMemcpyAsync(m.hbuf + static_cast<int64_t>(2) * Mx * H, hidden, static_cast<size_t>(n) * H * 4,
                                    hipMemcpyHostToDevice, stream()));
        for (int t = 0; t < n; ++t) hrow[t] = 2 * Mx + t;
        return 0;
    }
    const int avail = m.keep_rows.empty() ? m.hid_n : static_cast<int>(m.keep_rows.size());
    GV_REQUIRE(n <= avail, std::string(who) + ": no hidden rows given and the last verify left fewer than n");
    for (int t = 0; t < n; ++t) hrow[t] = m.keep_rows.empty() ? t : m.keep_rows[static_cast<size_t>(t)];
    return 0;
}

// The pass's launches on the model's stream (the step parameters: sp_mtp, swapped in for the layer's launches)
int mtp_launches(Model &m, int n, bool head, hipStream_t st) {
    const auto &c = m.c;
    const int H = c.hidden;
    const int64_t abH = act_halves(H);
    hipLaunchKernelGGL(mtp_in_kernel, dim3(n), dim3(256), 0, st, m.embed, m.sp, m.hbuf, m.mtp_pre_e, m.mtp_pre_h, c.eps,
                       m.mtp_act, act_halves(2 * static_cast<int64_t>(H)));
    GV_CHECK_HIP(hipGetLastError());
    if (gemv_q4(m.mtp_fc, m.mtp_act, act_halves(2 * static_cast<int64_t>(H)), n, gemv_out(m.x, H, m.mtp_fc.global), st) != 0)
        return -1;
    const LayerW &L = m.layers[static_cast<size_t>(c.n_layers)];
    if (quantize_act(m.x, H, n, H, L.in_norm, c.eps, m.act_h, abH, nullptr, 0, st) != 0) return -1;
    int ncls = 0;
    const int *cls = layer_classes(ncls);
    for (int i = 0; i < ncls; ++i)
        if (run_class(m, cls[i], c.n_layers, n, st) != 0) return -1;
    if (!head) return 0;
    const Q4 &hw = m.draft_head.rows > 0 ? m.draft_head : m.lm_head;
    if (gemv_q4(hw, m.act_h + static_cast<int64_t>(n - 1) * abH, abH, 1, gemv_out(m.mtp_logits, hw.rows, hw.global), st) != 0)
        return -1;
    auto *pa = static_cast<PickArea *>(m.pick);
    const int rows = static_cast<int>(hw.rows);
    hipLaunchKernelGGL(pick_max_kernel, dim3(kPickWgs), dim3(kPickThreads), 0, st, m.mtp_logits, rows, pa);
    hipLaunchKernelGGL(pick_sum_kernel, dim3(kPickWgs), dim3(kPickThreads), 0, st, m.mtp_logits, rows,
                       m.draft_head.rows > 0 ? m.draft_ids : nullptr, pa);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

// the pass's launches with the MTP step parameters swapped in: directly, or as the (rows, head) graph (captured on
// the second use; every parameter is read from device memory, so one graph serves every position and token)
int mtp_run(Model &m, int n, bool head, hipStream_t st) {
    StepParams *saved = m.sp;
    m.sp = m.sp_mtp;
    int rc = 0;
    bool &seen = m.mtp_seen[n][head ? 1 : 0];
    hipGraphExec_t &ge = m.mtp_graphs[n][head ? 1 : 0];
    if (!m.use_graphs || m.timed_class >= 0 || !seen) {
        seen = true;
        rc = mtp_launches(m, n, head, st);
    } else {
        if (!ge) {
            hipGraph_t graph = nullptr;
            if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
                m.sp = saved;
                GV_REQUIRE(false, "MTP pass: graph capture failed to start");
            }
            rc = mtp_launches(m, n, head, st);
            const hipError_t e = hipStreamEndCapture(st, &graph);
            if (rc == 0 && (e != hipSuccess || !graph)) rc = -1, set_error("MTP pass: graph capture failed");
            if (rc == 0 && hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0) != hipSuccess)
                rc = -1, ge = nullptr, set_error("MTP pass: graph instantiate failed");
            if (graph) (void)hipGraphDestroy(graph);
        }
        if (rc == 0 && hipGraphLaunch(ge, st) != hipSuccess) rc = -1, set_error("MTP pass: graph launch failed");
    }
    m.sp = saved;
    return rc;
}

// the pass, then its result (the draft and its probability, with the fused launches' error flag) in one wait
int mtp_pass(Model &m, int n, bool head) {
    hipStream_t st = stream();
    if (use_act_mode(m.c.exact) != 0) return -1;
    if (mtp_run(m, n, head, st) != 0) return -1;
    const auto *pa = static_cast<const PickArea *>(m.pick);
    if (head) GV_CHECK_HIP(hipMemcpyAsync(m.pick_host, &pa->draft, 8, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipMemcpyAsync(m.pick_host + 2, m.err, 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    GV_REQUIRE(m.pick_host[2] == 0, "MTP pass: a fused launch's wait for its producers ran out (the results are invalid)");
    if (head) m.mtp_last_n = n;
    return 0;
}

int mtp_result(Model &m, int32_t *draft, float *prob) {
    if (draft) *draft = m.pick_host[0];
    if (prob) *prob = __builtin_bit_cast(float, m.pick_host[1]);
    return 0;
}

void drop_head_graphs(Model &m) {   // (the head changed: the passes with a head are captured again)
    for (int n = 0; n <= kMaxRows; ++n) {
        if (m.mtp_graphs[n][1]) (void)hipGraphExecDestroy(m.mtp_graphs[n][1]);
        m.mtp_graphs[n][1] = nullptr;
        m.mtp_seen[n][1] = false;
    }
}

}  // namespace

GV_ACT_MODE_SETTER(act_mode_set_mtp)

int mtp_alloc(Model &m) {
    const auto &c = m.c;
    const int64_t H = c.hidden, Mx = c.max_rows;
    auto *fc = static_cast<uint8_t *>(mtp_dalloc(m, q4_code_bytes(H, 2 * H) + q4_scale_bytes(H, 2 * H)));
    auto *f = static_cast<float *>(mtp_dalloc(m, static_cast<size_t>(3 * H + 3 * Mx * H) * 4));
    m.mtp_act = static_cast<_Float16 *>(mtp_dalloc(m, static_cast<size_t>(Mx) * act_bytes(2 * H)));
    m.mtp_logits = static_cast<float *>(mtp_dalloc(m, static_cast<size_t>(c.vocab) * 4));
    m.sp_mtp = static_cast<StepParams *>(mtp_dalloc(m, sizeof(StepParams)));
    m.pick = mtp_dalloc(m, sizeof(PickArea));
    if (!fc || !f || !m.mtp_act || !m.mtp_logits || !m.sp_mtp || !m.pick) return -1;
    if (hipHostMalloc(reinterpret_cast<void **>(&m.pick_host), 16, hipHostMallocDefault) != hipSuccess) return -1;
    m.mtp_fc.codes = fc;
    m.mtp_fc.scales = fc + q4_code_bytes(H, 2 * H);
    m.mtp_fc.rows = H;
    m.mtp_fc.cols = 2 * H;
    m.mtp_norm = f, m.mtp_pre_e = f + H, m.mtp_pre_h = f + 2 * H, m.hbuf = f + 3 * H;
    if (hipMemset(f, 0, static_cast<size_t>(3 * H + 3 * Mx * H) * 4) != hipSuccess ||
        hipMemset(m.pick, 0, sizeof(PickArea)) != hipSuccess || hipMemset(fc, 0, q4_code_bytes(H, 2 * H) + q4_scale_bytes(H, 2 * H)) != hipSuccess)
        return -1;
    return 0;
}

void mtp_free(Model &m) {
    if (m.draft_mem) (void)hipFree(m.draft_mem);
    m.draft_mem = nullptr;
}

void mtp_release(Model &m) {
    mtp_free(m);
    for (auto &row : m.mtp_graphs)
        for (auto &ge : row)
            if (ge) (void)hipGraphExecDestroy(ge), ge = nullptr;
    if (m.pick_host) (void)hipHostFree(m.pick_host);
    m.pick_host = nullptr;
}

}  // namespace gv

using namespace gv;

extern "C" {

int gv_model_draft(gv_model *g, const int32_t *toks, int n, int pos, const float *hidden, int32_t *draft, float *prob) {
    GV_REQUIRE(g && toks, "gv_model_draft: null pointer");
    Model &m = model_of(g);
    GV_REQUIRE(m.has_mtp, "gv_model_draft: the model has no MTP layer");
    GV_REQUIRE(n >= 1 && n <= m.c.max_rows, "gv_model_draft: 1 <= n <= max_rows");
    int hrow[kMaxRows];
    if (mtp_hidden_rows(m, n, hidden, hrow, "gv_model_draft") != 0) return -1;
    if (mtp_params(m, toks, n, pos, hrow, "gv_model_draft") != 0) return -1;
    if (mtp_pass(m, n, true) != 0) return -1;
    return mtp_result(m, draft, prob);
}

int gv_model_draft_next(gv_model *g, int32_t tok, int pos, int32_t *draft, float *prob) {
    GV_REQUIRE(g, "gv_model_draft_next: null model");
    Model &m = model_of(g);
    GV_REQUIRE(m.has_mtp, "gv_model_draft_next: the model has no MTP layer");
    GV_REQUIRE(m.mtp_last_n > 0, "gv_model_draft_next: no MTP pass to go on from");
    const int hrow[1] = {m.c.max_rows + m.mtp_last_n - 1};   // the last pass's last row after mtp.norm
    if (mtp_params(m, &tok, 1, pos, hrow, "gv_model_draft_next") != 0) return -1;
    if (mtp_pass(m, 1, true) != 0) return -1;
    return mtp_result(m, draft, prob);
}

int gv_model_draft_chain(gv_model *g, const int32_t *toks, int n, int pos, const float *hidden, int kmax, float pmin,
                         int32_t *drafts, float *probs, int *count) {
    GV_REQUIRE(g && toks && drafts && count, "gv_model_draft_chain: null pointer");
    GV_REQUIRE(kmax >= 2, "gv_model_draft_chain: kmax >= 2 (the token and at least one draft)");
    Model &m = model_of(g);
    *count = 0;
    float p = 0.0f;
    if (gv_model_draft(g, toks, n, pos, hidden, &drafts[0], &p) != 0) return -1;
    if (probs) probs[0] = p;
    int k = 1;   // drafts so far; the verify batch is the token and them: k + 1 rows
    int q = pos + n;   // the MTP position the next chained draft takes
    // geode.cpp:310-317: chained while the batch is short of kmax, the last draft sure enough and the batch (and the
    // MTP row) still inside the context
    while (k + 1 < kmax && p >= pmin && m.pos + k + 2 < m.c.max_ctx && q < m.c.max_ctx) {
        int32_t d = 0;
        if (gv_model_draft_next(g, drafts[k - 1], q, &d, &p) != 0) return -1;
        if (p < pmin) break;   // too unsure to be worth its experts
        drafts[k] = d;
        if (probs) probs[k] = p;
        ++k;
        ++q;
    }
    *count = k;
    return 0;
}

int gv_model_mtp_fill(gv_model *g, const int32_t *toks, int n, int pos, const float *hidden) {
    GV_REQUIRE(g && toks && n >= 1, "gv_model_mtp_fill: bad arguments");
    Model &m = model_of(g);
    GV_REQUIRE(m.has_mtp, "gv_model_mtp_fill: the model has no MTP layer");
    const int Mx = m.c.max_rows, H = m.c.hidden;
    GV_REQUIRE(hidden || n <= Mx, "gv_model_mtp_fill: more than max_rows rows need their hidden rows given");
    for (int t0 = 0; t0 < n; t0 += Mx) {
        const int k = std::min(Mx, n - t0);
        int hrow[kMaxRows];
        if (mtp_hidden_rows(m, k, hidden ? hidden + static_cast<int64_t>(t0) * H : nullptr, hrow, "gv_model_mtp_fill") != 0)
            return -1;
        if (mtp_params(m, toks + t0, k, pos + t0, hrow, "gv_model_mtp_fill") != 0) return -1;
        if (mtp_pass(m, k, false) != 0) return -1;
    }
    return 0;
}

int gv_model_set_draft_vocab(gv_model *g, const int32_t *ids, int n) {
    GV_REQUIRE(g && n >= 0 && (n == 0 || ids), "gv_model_set_draft_vocab: bad arguments");
    Model &m = model_of(g);
    const auto &c = m.c;
    GV_REQUIRE(n <= c.vocab, "gv_model_set_draft_vocab: more ids than the vocabulary");
    for (int i = 0; i < n; ++i) GV_REQUIRE(ids[i] >= 0 && ids[i] < c.vocab, "gv_model_set_draft_vocab: id out of range");
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    mtp_free(m);
    drop_head_graphs(m);
    m.draft_head = Q4{};
    m.draft_ids = nullptr;
    if (n == 0) return 0;
    const int64_t H = c.hidden;
    const size_t cb = q4_code_bytes(n, H), sb = q4_scale_bytes(n, H);
    GV_CHECK_HIP(hipMalloc(&m.draft_mem, cb + sb + static_cast<size_t>(n) * 4));
    GV_CHECK_HIP(hipMemsetAsync(m.draft_mem, 0, cb + sb, stream()));   // the last tile's missing rows: zero
    auto *dids = reinterpret_cast<int32_t *>(m.draft_mem + cb + sb);
    GV_CHECK_HIP(hipMemcpyAsync(dids, ids, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, stream()));
    const int64_t items = static_cast<int64_t>(n) * (H / 8);
    hipLaunchKernelGGL(draft_rows_kernel, dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0, stream(),
                       m.lm_head, dids, n, m.draft_mem, m.draft_mem + cb);
    GV_CHECK_HIP(hipGetLastError());
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    m.draft_head.codes = m.draft_mem;
    m.draft_head.scales = m.draft_mem + cb;
    m.draft_head.rows = n;
    m.draft_head.cols = H;
    m.draft_head.global = m.lm_head.global;
    m.draft_ids = dids;
    return 0;
}

int gv_model_hidden(const gv_model *g, float *out, int max_rows) {
    GV_REQUIRE(g && out, "gv_model_hidden: null pointer");
    Model &m = model_of(const_cast<gv_model *>(g));
    GV_REQUIRE(m.has_mtp, "gv_model_hidden: the model has no MTP layer (it keeps no hidden rows)");
    const int k = std::min(m.hid_n, max_rows);
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    if (k > 0) GV_CHECK_HIP(hipMemcpy(out, m.hbuf, static_cast<size_t>(k) * m.c.hidden * 4, hipMemcpyDeviceToHost));
    return k;
}

int gv_model_draft_logits(const gv_model *g, float *out) {
    GV_REQUIRE(g && out, "gv_model_draft_logits: null pointer");
    Model &m = model_of(const_cast<gv_model *>(g));
    GV_REQUIRE(m.has_mtp && m.mtp_last_n > 0, "gv_model_draft_logits: no MTP pass yet");
    GV_CHECK_HIP(hipStreamSynchronize(stream()));
    const int64_t rows = head_rows(m);
    GV_CHECK_HIP(hipMemcpy(out, m.mtp_logits, static_cast<size_t>(rows) * 4, hipMemcpyDeviceToHost));
    return static_cast<int>(rows);
}

}  // extern "C"
