// sample.hip - the sampler and the two acceptance rules on the GPU.
//
//   Sampler::sample       sampler.cpp:16-50        T <= 0: the first argmax. Else the candidates (top_k, else the
//                                                   top `cap` = 1024, ties to the lower index) by logit descending,
//                                                   e = exp((l - max) / T) in float, their sum in double, top-p the
//                                                   smallest prefix whose probability reaches p, r = kept x u, the
//                                                   first candidate where r - (e_0 + .. + e_i) <= 0.
//   sample-and-match      geode.cpp:318-374        each verified row sampled with its own uniform; a draft stands
//                                                   while the row before samples exactly it.
//   textbook rule         (Leviathan et al. 2023, Alg. 1; not in the reference) accept d ~ q with probability
//                                                   min(1, p(d) / q(d)); at the first rejection a token from
//                                                   max(0, p - q) by inverse CDF in index order; a bonus from p_k
//                                                   when every draft stands.
//
// Per row, topk_kernel selects the K candidates with a three-pass radix select on order-preserving 32-bit keys
// (11 + 11 + 10 bits, LDS histograms), collects them (ties at the threshold to the lower index) and sorts them with
// a bitonic sort in LDS; nucleus_kernel computes e, the top-p prefix, the kept mass and the draw; the acceptance
// kernels walk the rows. The double sums run as parallel scans: they differ from the reference's sequential sums in
// the last bits (~1e-16 relative), which moves a decision only when a uniform or top_p falls that close to a
// boundary; expf is the device's (within 1 ulp of glibc's).
#include <algorithm>
#include <climits>
#include <vector>

#include "../../include/geode_verify.h"
#include "common.hpp"
#include "kernels.hpp"

namespace gv {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kMaxCand = 16384;   // candidates a row can keep (the full-vocabulary nucleus must fit)
constexpr int kRowBatch = 8;      // a row's values a thread loads at once in the full-row passes

// float -> a key whose unsigned order is the float order (-0 taken as +0: equal floats, equal keys)
__device__ inline uint32_t fkey(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float key_val(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

template <typename T>
__device__ inline T wave_incl_scan(T v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        const T u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}

// exclusive scan over the workgroup (thread order); tot: the total; tmp: LDS of 16 T
template <typename T>
__device__ inline T block_excl_scan(T v, T *tmp, T &tot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const T incl = wave_incl_scan(v);
    __syncthreads();   // tmp may still be read by an earlier scan
    if (lane == 63) tmp[wave] = incl;
    __syncthreads();
    T base = 0, all = 0;
    for (int w = 0; w < nw; ++w) {
        if (w < wave) base += tmp[w];
        all += tmp[w];
    }
    tot = all;
    return base + incl - v;
}

template <typename T>
__device__ inline T block_sum(T v, T *tmp) {
    T tot;
    (void)block_excl_scan(v, tmp, tot);
    return tot;
}

// The K largest of a row (K <= KP, KP a power of two), by value descending, ties to the lower index: keys to okey,
// indices to oidx. full_sum: also the sum over the whole row of exp((l - max) / T) in double (the full-vocabulary
// nucleus's denominator) to osum.
template <int KP>
__global__ __launch_bounds__(kSelThreads) void topk_kernel(const float *__restrict__ x, int64_t ldx, int V, int K,
                                                            float T, int full_sum, uint32_t *__restrict__ okey,
                                                            int32_t *__restrict__ oidx, int64_t ostride,
                                                            double *__restrict__ osum) {
    extern __shared__ uint64_t comp[];   // [KP] (key << 32) | (~index): descending = value desc, index asc
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t tmp_u[16];
    __shared__ double tmp_d[16];
    __shared__ uint32_t s_prefix, s_mask, s_above, s_need, s_maxkey, s_cnt, s_bin, s_add, s_bincnt;
    const float *row = x + static_cast<int64_t>(blockIdx.x) * ldx;
    const int tid = threadIdx.x, nthr = blockDim.x;
    if (tid == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_above = 0;
        s_need = static_cast<uint32_t>(K);
        s_maxkey = 0;
        s_cnt = 0;
    }
    __syncthreads();
    constexpr int kShift[3] = {21, 10, 0}, kWidth[3] = {11, 11, 10};
    uint32_t cnt_eq = 0;
#pragma unroll
    for (int p = 0; p < 3; ++p) {
        const int sh = kShift[p], nb = 1 << kWidth[p];
        for (int i = tid; i < nb; i += nthr) hist[i] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask, need = s_need;
        uint32_t mk = 0;
        for (int i0 = tid; i0 < V; i0 += kRowBatch * nthr) {   // kRowBatch loads in flight a thread
            float v[kRowBatch];
#pragma unroll
            for (int u = 0; u < kRowBatch; ++u) v[u] = row[min(i0 + u * nthr, V - 1)];
#pragma unroll
            for (int u = 0; u < kRowBatch; ++u) {   // (no branch before the uses: no load sinks into one)
                const bool in = i0 + u * nthr < V;
                const uint32_t k = fkey(v[u]);
                if (p == 0) mk = max(mk, in ? k : 0u);
                if (in && (k & mask) == prefix) atomicAdd(&hist[(k >> sh) & (nb - 1)], 1u);
            }
        }
        if (p == 0) atomicMax(&s_maxkey, mk);
        __syncthreads();
        // from the top bin down: the bin where the count reaches need (thread t: bins nb-1-2t, nb-2-2t)
        const int r0 = 2 * tid, r1 = 2 * tid + 1;
        const uint32_t c0 = r1 < nb ? hist[nb - 1 - r0] : 0u, c1 = r1 < nb ? hist[nb - 1 - r1] : 0u;
        uint32_t tot;
        const uint32_t ex = block_excl_scan(c0 + c1, tmp_u, tot);
        if (r1 < nb) {
            if (ex < need && ex + c0 >= need) {
                s_bin = static_cast<uint32_t>(nb - 1 - r0);
                s_add = ex;
                s_bincnt = c0;
            } else if (ex + c0 < need && ex + c0 + c1 >= need) {
                s_bin = static_cast<uint32_t>(nb - 1 - r1);
                s_add = ex + c0;
                s_bincnt = c1;
            }
        }
        __syncthreads();
        if (tid == 0) {
            s_prefix = prefix | (s_bin << sh);
            s_mask = mask | (static_cast<uint32_t>(nb - 1) << sh);
            s_above += s_add;
            s_need = need - s_add;
        }
        cnt_eq = s_bincnt;
        __syncthreads();
    }
    const uint32_t tau = s_prefix, above = s_above, need_eq = s_need;
    const bool all_eq = cnt_eq == need_eq;
    const float mx = key_val(s_maxkey);
    double esum = 0.0;
    for (int i0 = tid; i0 < V; i0 += kRowBatch * nthr) {
        float v[kRowBatch];
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) v[u] = row[min(i0 + u * nthr, V - 1)];
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
            const int i = i0 + u * nthr;
            const bool in = i < V;
            const float f = v[u];
            const uint32_t k = fkey(f);
            if (full_sum) esum += in ? static_cast<double>(expf(__fdiv_rn(__fsub_rn(f, mx), T))) : 0.0;
            if (in && (k > tau || (all_eq && k == tau))) {
                const uint32_t slot = atomicAdd(&s_cnt, 1u);
                if (slot < static_cast<uint32_t>(K))
                    comp[slot] = (static_cast<uint64_t>(k) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
            }
        }
    }
    if (!all_eq) {   // ties at the threshold beyond what is needed: the lowest indices, in index order
        __syncthreads();
        const int ch = (V + nthr - 1) / nthr, b0 = tid * ch, b1 = min(V, b0 + ch);
        uint32_t c = 0;
        for (int i = b0; i < b1; ++i) c += fkey(row[i]) == tau;
        uint32_t tot;
        uint32_t r = block_excl_scan(c, tmp_u, tot);
        for (int i = b0; i < b1 && r < need_eq && above + r < static_cast<uint32_t>(K); ++i)
            if (fkey(row[i]) == tau) {
                comp[above + r] = (static_cast<uint64_t>(tau) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
                ++r;
            }
    }
    for (int i = K + tid; i < KP; i += nthr) comp[i] = 0;
    if (full_sum) {
        const double s = block_sum(esum, tmp_d);
        if (tid == 0) osum[blockIdx.x] = s;
    }
    __syncthreads();
    // bitonic sort, descending. Pair i of a stage of stride s <= 64 has both elements in [128 (i / 64), + 128): a
    // wave's 64 consecutive pairs keep the same 128 elements from one such stage to the next, so between two of them
    // the wave only waits for its own LDS writes; a workgroup barrier follows every other stage.
    for (int size = 2; size <= KP; size <<= 1)
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int i = tid; i < KP / 2; i += nthr) {
                const int lo = 2 * stride * (i / stride) + (i % stride), hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t a = comp[lo], b = comp[hi];
                if ((a < b) == desc) {
                    comp[lo] = b;
                    comp[hi] = a;
                }
            }
            const int next = stride > 1 ? stride / 2 : size;   // the next stage's stride (size * 2 / 2)
            if (stride <= 64 && next <= 64 && !(stride == 1 && size == KP)) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else {
                __syncthreads();
            }
        }
    uint32_t *ok = okey + static_cast<int64_t>(blockIdx.x) * ostride;
    int32_t *oi = oidx + static_cast<int64_t>(blockIdx.x) * ostride;
    for (int i = tid; i < K; i += nthr) {
        ok[i] = static_cast<uint32_t>(comp[i] >> 32);
        oi[i] = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(comp[i]));
    }
}

// Per row: e_i = exp((l_i - max) / T) of its K sorted candidates (to oe), the sum (osum[row] when given: the whole
// row's; else the candidates'), keep = the top-p prefix (K when top_p >= 1; *short_out set when the candidates
// run out first), kept = e_0 + .. + e_{keep-1}, and the draw of u[row]: the first i < keep where kept u <= e_0 + .. +
// e_i (else keep - 1), its position to opos and index to opick.
__global__ __launch_bounds__(kSelThreads) void nucleus_kernel(const uint32_t *__restrict__ okey,
                                                               const int32_t *__restrict__ oidx, int64_t cs, int K,
                                                               const double *__restrict__ osum, float T, float top_p,
                                                               const double *__restrict__ u, float *__restrict__ oe,
                                                               int *__restrict__ okeep, double *__restrict__ okept,
                                                               int *__restrict__ opos, int32_t *__restrict__ opick,
                                                               int *__restrict__ short_out) {
    __shared__ double tmp_d[16];
    __shared__ int s_first;
    const int row = blockIdx.x, tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t *key = okey + static_cast<int64_t>(row) * cs;
    float *e = oe + static_cast<int64_t>(row) * cs;
    const float mx = key_val(key[0]);
    double part = 0.0;
    for (int i = tid; i < K; i += nthr) {
        const float v = expf(__fdiv_rn(__fsub_rn(key_val(key[i]), mx), T));
        e[i] = v;
        part += static_cast<double>(v);
    }
    const double cand_sum = block_sum(part, tmp_d);   // (its syncs also publish e)
    const double sum = osum ? osum[row] : cand_sum;
    // keep: the first i where (e_0 + .. + e_i) / sum ... as the reference: acc += e_i / sum, acc >= top_p
    int keep = K;
    if (top_p < 1.0f) {
        if (tid == 0) s_first = K;
        double carry = 0.0;
        for (int c0 = 0; c0 < K; c0 += nthr) {
            const int i = c0 + tid;
            const double t = i < K ? static_cast<double>(e[i]) / sum : 0.0;
            double tot;
            const double acc = carry + block_excl_scan(t, tmp_d, tot) + t;
            if (i < K && acc >= static_cast<double>(top_p)) atomicMin(&s_first, i);
            carry += tot;
            __syncthreads();
            if (s_first < K) break;
        }
        keep = s_first < K ? s_first + 1 : K;
        if (tid == 0 && short_out && s_first >= K) atomicOr(short_out, 1);
    }
    // kept and the draw
    __syncthreads();   // every thread has read s_first
    if (tid == 0) s_first = INT32_MAX;
    double carry = 0.0;
    for (int c0 = 0; c0 < keep; c0 += nthr) {   // kept: the sum of the first keep
        const int i = c0 + tid;
        const double t = i < keep ? static_cast<double>(e[i]) : 0.0;
        carry += block_sum(t, tmp_d);
    }
    const double kept = carry;
    const double r = kept * u[row];
    carry = 0.0;
    for (int c0 = 0; c0 < keep; c0 += nthr) {
        const int i = c0 + tid;
        const double t = i < keep ? static_cast<double>(e[i]) : 0.0;
        double tot;
        const double acc = carry + block_excl_scan(t, tmp_d, tot) + t;
        if (i < keep && r - acc <= 0.0) atomicMin(&s_first, i);
        carry += tot;
        __syncthreads();
        if (s_first != INT32_MAX) break;
    }
    __syncthreads();
    if (tid == 0) {
        const int at = s_first != INT32_MAX ? s_first : keep - 1;   // rounding past the end: the last kept
        okeep[row] = keep;
        okept[row] = kept;
        opos[row] = at;
        opick[row] = oidx[static_cast<int64_t>(row) * cs + at];
    }
}

// sample-and-match over the sampled rows (geode.cpp:331-350): out = the stood drafts then the first sampled token
// that is no draft; a draft stands only if it is no stop token either (stop[0..n_stop)); res = {emitted, kept}
__global__ void match_kernel(const int32_t *__restrict__ pick, const int32_t *__restrict__ batch, int n,
                             const int32_t *__restrict__ stop, int n_stop, int32_t *__restrict__ out,
                             int *__restrict__ res) {
    if (threadIdx.x != 0) return;
    int emitted = 0, kept = 1;
    for (int i = 0; i < n; ++i) {
        out[emitted++] = pick[i];
        bool is_stop = false;
        for (int j = 0; j < n_stop; ++j) is_stop |= stop[j] == pick[i];
        if (i + 1 < n && pick[i] == batch[i + 1] && !is_stop) {
            ++kept;
            continue;
        }
        break;
    }
    res[0] = emitted;
    res[1] = kept;
}

// The presence penalty of the generate loop (geode.cpp:236-255) on the verified rows, in place: row i (a workgroup)
// loses `penalty` at each of the answer's seen tokens (distinct) and at each draft batch[j], 1 <= j <= i, that is
// new (fresh[j]: in neither `seen` nor an earlier draft), the tokens rows 0..i-1 sampled if their drafts stood (a
// row after a fallen draft is never used). One subtraction a token, as the reference's once-each list.
__global__ void penalty_kernel(float *__restrict__ logits, int64_t ld, const int32_t *__restrict__ seen, int n_seen,
                               const int32_t *__restrict__ batch, const int32_t *__restrict__ fresh, float penalty) {
    float *lg = logits + static_cast<int64_t>(blockIdx.x) * ld;
    for (int j = threadIdx.x; j < n_seen; j += blockDim.x) lg[seen[j]] -= penalty;
    for (int j = 1 + static_cast<int>(threadIdx.x); j <= static_cast<int>(blockIdx.x); j += blockDim.x)
        if (fresh[j]) lg[batch[j]] -= penalty;
}

__global__ void first_kernel(const int32_t *__restrict__ idx, int64_t cs, int rows, int32_t *__restrict__ pick) {
    for (int r = threadIdx.x; r < rows; r += blockDim.x) pick[r] = idx[static_cast<int64_t>(r) * cs];
}

struct RowSet {   // the nucleus outputs of a set of rows
    const uint32_t *key;
    const int32_t *idx;
    const float *e;
    const int *keep;
    const double *kept;
    const int *pos;
    const int32_t *pick;
    int64_t cs;
};

// The textbook rule over k drafts (target rows 0..k, draft rows 0..k-1), one workgroup. qq: a zeroed device array
// of V doubles (left zeroed). res[0] = emitted.
__global__ __launch_bounds__(kSelThreads) void textbook_kernel(RowSet P, RowSet Q, int k, int greedy,
                                                               const float *__restrict__ u_acc, float u_res,
                                                               double *__restrict__ qq, int32_t *__restrict__ out,
                                                               int *__restrict__ res) {
    extern __shared__ uint64_t srt[];   // [kMaxCand] (index << 32) | slot, for the residual in index order
    __shared__ double tmp_d[16];
    __shared__ int s_pd_pos, s_first;
    const int tid = threadIdx.x, nthr = blockDim.x;
    int emitted = 0;
    bool all_stood = true;
    for (int i = 0; i < k; ++i) {
        if (greedy) {   // argmax = the first candidate (ties to the lower index, as max_element)
            const int y = P.idx[i * P.cs], d = Q.idx[i * Q.cs];
            if (tid == 0) out[emitted] = y;
            ++emitted;
            if (y != d) {
                all_stood = false;
                break;
            }
            continue;
        }
        const int d = Q.pick[i];
        const double qd = static_cast<double>(Q.e[i * Q.cs + Q.pos[i]]) / Q.kept[i];
        if (tid == 0) s_pd_pos = -1;
        __syncthreads();
        const int kp = P.keep[i];
        for (int j = tid; j < kp; j += nthr)
            if (P.idx[i * P.cs + j] == d) s_pd_pos = j;
        __syncthreads();
        const double pd = s_pd_pos >= 0 ? static_cast<double>(P.e[i * P.cs + s_pd_pos]) / P.kept[i] : 0.0;
        if (static_cast<double>(u_acc[i]) * qd < pd) {   // accepted with probability min(1, p/q)
            if (tid == 0) out[emitted] = d;
            ++emitted;
            continue;
        }
        // rejected: a token from max(0, p - q), normalized, by inverse CDF in index order
        const int kq = Q.keep[i];
        for (int j = tid; j < kq; j += nthr)
            qq[Q.idx[i * Q.cs + j]] = static_cast<double>(Q.e[i * Q.cs + j]) / Q.kept[i];
        __syncthreads();
        int np = 1;
        while (np < kp) np <<= 1;
        for (int j = tid; j < np; j += nthr)
            srt[j] = j < kp ? (static_cast<uint64_t>(static_cast<uint32_t>(P.idx[i * P.cs + j])) << 32) |
                                  static_cast<uint32_t>(j)
                            : ~0ull;
        __syncthreads();
        for (int size = 2; size <= np; size <<= 1)   // ascending by index
            for (int stride = size / 2; stride > 0; stride >>= 1) {
                for (int j = tid; j < np / 2; j += nthr) {
                    const int lo = 2 * stride * (j / stride) + (j % stride), hi = lo + stride;
                    const bool asc = (lo & size) == 0;
                    const uint64_t a = srt[lo], b = srt[hi];
                    if ((a > b) == asc) {
                        srt[lo] = b;
                        srt[hi] = a;
                    }
                }
                __syncthreads();
            }
        // residual weights in index order, their total, and the inverse CDF
        auto resid = [&](int j) -> double {
            if (j >= kp) return 0.0;
            const int slot = static_cast<int>(srt[j] & 0xFFFFFFFFu), x = static_cast<int>(srt[j] >> 32);
            const double pp = static_cast<double>(P.e[i * P.cs + slot]) / P.kept[i];
            return fmax(0.0, pp - qq[x]);
        };
        double total = 0.0;
        for (int c0 = 0; c0 < kp; c0 += nthr) total += block_sum(resid(c0 + tid), tmp_d);
        int pick;
        if (!(total > 0.0)) {
            pick = P.pick[i];   // the row's own draw; the caller drew target rows with u_res
        } else {
            const double goal = static_cast<double>(u_res) * total;
            if (tid == 0) s_first = kp;
            double carry = 0.0;
            for (int c0 = 0; c0 < kp; c0 += nthr) {
                const int j = c0 + tid;
                const double t = resid(j);
                double tot;
                const double acc = carry + block_excl_scan(t, tmp_d, tot) + t;
                if (j < kp && t > 0.0 && acc >= goal) atomicMin(&s_first, j);
                carry += tot;
                __syncthreads();
                if (s_first < kp) break;
            }
            __syncthreads();
            int j = s_first;
            if (j >= kp) {   // rounding left the goal past the end: the last positive weight
                j = kp - 1;
                while (j > 0 && !(resid(j) > 0.0)) --j;
            }
            pick = static_cast<int>(srt[j] >> 32);
        }
        __syncthreads();   // every thread is done reading qq
        for (int j = tid; j < kq; j += nthr) qq[Q.idx[i * Q.cs + j]] = 0.0;   // leave qq zeroed
        if (tid == 0) out[emitted] = pick;
        ++emitted;
        if (tid == 0) res[0] = emitted;
        return;
    }
    if (all_stood) {   // every draft stood: the bonus token from the last target row
        if (tid == 0) out[emitted] = greedy ? P.idx[k * P.cs] : P.pick[k];
        ++emitted;
    }
    if (tid == 0) res[0] = emitted;
}

// ---------------------------------------------------------------- host side
struct Workspace {
    void *p = nullptr;
    size_t n = 0;
    void *get(size_t want) {
        if (want <= n) return p;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        if (hipMalloc(&p, want) != hipSuccess) return nullptr;
        n = want;
        return p;
    }
};

struct Nuclei {   // device arrays for R rows of up to C candidates
    uint32_t *key;
    int32_t *idx;
    float *e;
    double *sum, *kept, *u;
    int *keep, *pos, *flag;
    int32_t *pick;
    int64_t cs;
    RowSet rows(int r0) const {
        return RowSet{key + r0 * cs, idx + r0 * cs, e + r0 * cs, keep + r0, kept + r0, pos + r0, pick + r0, cs};
    }
};

size_t nuclei_bytes(int R, int C) {
    return static_cast<size_t>(R) * C * (4 + 4 + 4) + static_cast<size_t>(R) * (8 * 3 + 4 * 3 + 4) + 64;
}

Nuclei carve(void *base, int R, int C) {
    char *p = static_cast<char *>(base);
    Nuclei n;
    n.cs = C;
    n.key = reinterpret_cast<uint32_t *>(p);
    p += static_cast<size_t>(R) * C * 4;
    n.idx = reinterpret_cast<int32_t *>(p);
    p += static_cast<size_t>(R) * C * 4;
    n.e = reinterpret_cast<float *>(p);
    p += static_cast<size_t>(R) * C * 4;
    n.sum = reinterpret_cast<double *>(p);
    p += static_cast<size_t>(R) * 8;
    n.kept = reinterpret_cast<double *>(p);
    p += static_cast<size_t>(R) * 8;
    n.u = reinterpret_cast<double *>(p);
    p += static_cast<size_t>(R) * 8;
    n.keep = reinterpret_cast<int *>(p);
    p += static_cast<size_t>(R) * 4;
    n.pos = reinterpret_cast<int *>(p);
    p += static_cast<size_t>(R) * 4;
    n.pick = reinterpret_cast<int32_t *>(p);
    p += static_cast<size_t>(R) * 4;
    n.flag = reinterpret_cast<int *>(p);
    return n;
}

template <int KP>
int launch_topk(const float *x, int64_t ldx, int rows, int V, int K, float T, int full, const Nuclei &n,
                hipStream_t st) {
    static int granted = 0;
    const size_t lds = static_cast<size_t>(KP) * 8;
    if (lds_grant(reinterpret_cast<const void *>(&topk_kernel<KP>), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(topk_kernel<KP>, dim3(rows), dim3(kSelThreads), lds, st, x, ldx, V, K, T, full, n.key, n.idx,
                       n.cs, n.sum);
    GV_CHECK_HIP(hipGetLastError());
    return 0;
}

int topk(const float *x, int64_t ldx, int rows, int V, int K, float T, int full, const Nuclei &n, hipStream_t st) {
    if (K <= 1024) return launch_topk<1024>(x, ldx, rows, V, K, T, full, n, st);
    if (K <= 4096) return launch_topk<4096>(x, ldx, rows, V, K, T, full, n, st);
    return launch_topk<kMaxCand>(x, ldx, rows, V, K, T, full, n, st);
}

// The nuclei of `rows` rows with uniforms u (host): candidates K = top_k, else cap, else (cap = 0, the full
// vocabulary) the smallest of 4096 / 16384 that holds the top-p prefix. T <= 0: K = 1 (the first argmax).
int nuclei(const float *x, int64_t ldx, int rows, int V, float T, float top_p, int top_k, int cap, const double *u,
           const Nuclei &n, hipStream_t st) {
    GV_REQUIRE(x && rows >= 1 && V >= 1, "sampler: bad arguments");
    if (T <= 0.0f) {   // the first argmax: the top candidate (ties to the lower index)
        if (topk(x, ldx, rows, V, 1, 1.0f, 0, n, st) != 0) return -1;
        hipLaunchKernelGGL(first_kernel, dim3(1), dim3(64), 0, st, n.idx, n.cs, rows, n.pick);
        GV_CHECK_HIP(hipGetLastError());
        return 0;
    }
    GV_CHECK_HIP(hipMemcpyAsync(n.u, u, static_cast<size_t>(rows) * 8, hipMemcpyHostToDevice, st));
    const bool full = top_k <= 0 && cap <= 0;
    GV_REQUIRE(!full || top_p < 1.0f, "sampler: the full vocabulary needs top_p < 1 (the nucleus is sorted on the GPU)");
    for (int K0 : {4096, kMaxCand}) {
        int K = top_k > 0 ? std::min(top_k, V) : (cap > 0 ? std::min(cap, V) : std::min(K0, V));
        GV_REQUIRE(K <= kMaxCand, "sampler: at most 16384 candidates");
        GV_CHECK_HIP(hipMemsetAsync(n.flag, 0, 4, st));
        if (topk(x, ldx, rows, V, K, T, full ? 1 : 0, n, st) != 0) return -1;
        hipLaunchKernelGGL(nucleus_kernel, dim3(rows), dim3(kSelThreads), 0, st, n.key, n.idx, n.cs, K,
                           full ? n.sum : nullptr, T, top_p, n.u, n.e, n.keep, n.kept, n.pos, n.pick, n.flag);
        GV_CHECK_HIP(hipGetLastError());
        if (!full) return 0;
        int flag = 0;
        GV_CHECK_HIP(hipMemcpyAsync(&flag, n.flag, 4, hipMemcpyDeviceToHost, st));
        GV_CHECK_HIP(hipStreamSynchronize(st));
        if (!flag || K == V) return 0;
        GV_REQUIRE(K0 != kMaxCand, "sampler: the top-p nucleus holds more than 16384 candidates");
    }
    return 0;
}

Workspace &ws() {
    static Workspace w;
    return w;
}

}  // namespace
}  // namespace gv

using namespace gv;

extern "C" {

int gv_sample_rows(const float *logits, int64_t ld, int rows, int V, float temperature, float top_p, int top_k,
                   int cap, const double *u, int32_t *out) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(logits && out && rows >= 1 && rows <= 64 && V >= 1 && ld >= V, "gv_sample_rows: bad arguments");
    GV_REQUIRE(temperature <= 0.0f || u, "gv_sample_rows: uniforms needed when temperature > 0");
    void *base = ws().get(nuclei_bytes(rows, kMaxCand));
    GV_REQUIRE(base, "gv_sample_rows: out of device memory");
    const Nuclei n = carve(base, rows, kMaxCand);
    const hipStream_t st = stream();
    if (nuclei(logits, ld, rows, V, temperature, top_p, top_k, cap, u, n, st) != 0) return -1;
    GV_CHECK_HIP(hipMemcpyAsync(out, n.pick, static_cast<size_t>(rows) * 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    return 0;
}

int gv_accept_match(const float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature,
                    float top_p, int top_k, int cap, const double *u, int32_t *out, int *kept) {
    // (no penalty: the rows are only read)
    return gv_accept_match_ex(const_cast<float *>(logits), ld, V, batch, n, temperature, top_p, top_k, cap, u, nullptr,
                              0, 0.0f, nullptr, 0, out, kept);
}

int gv_accept_match_ex(float *logits, int64_t ld, int V, const int32_t *batch, int n, float temperature, float top_p,
                       int top_k, int cap, const double *u, const int32_t *seen, int n_seen, float presence_penalty,
                       const int32_t *stop, int n_stop, int32_t *out, int *kept) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(logits && batch && out && n >= 1 && n <= 32 && V >= 1 && ld >= V, "gv_accept_match: bad arguments");
    GV_REQUIRE(temperature <= 0.0f || u, "gv_accept_match: uniforms needed when temperature > 0");
    GV_REQUIRE(n_seen >= 0 && (n_seen == 0 || seen) && n_seen <= V, "gv_accept_match: seen tokens");
    GV_REQUIRE(n_stop >= 0 && n_stop <= 1024 && (n_stop == 0 || stop), "gv_accept_match: at most 1024 stop tokens");
    const bool penalize = presence_penalty != 0.0f;
    // which drafts are new to the answer (one subtraction a token); seen must hold distinct tokens of the vocabulary
    std::vector<int32_t> fresh(33, 0);
    if (penalize) {
        std::vector<uint8_t> in(static_cast<size_t>(V), 0);
        for (int j = 0; j < n_seen; ++j) {
            GV_REQUIRE(seen[j] >= 0 && seen[j] < V && !in[static_cast<size_t>(seen[j])],
                       "gv_accept_match: seen tokens must be distinct tokens of the vocabulary");
            in[static_cast<size_t>(seen[j])] = 1;
        }
        for (int j = 1; j < n; ++j) {
            GV_REQUIRE(batch[j] >= 0 && batch[j] < V, "gv_accept_match: draft out of range");
            if (!in[static_cast<size_t>(batch[j])]) fresh[static_cast<size_t>(j)] = 1, in[static_cast<size_t>(batch[j])] = 1;
        }
    }
    const size_t nb = nuclei_bytes(n, kMaxCand);
    const size_t extra = (64 + 33 + static_cast<size_t>(n_stop) + (penalize ? static_cast<size_t>(n_seen) : 0)) * 4 + 256;
    char *base = static_cast<char *>(ws().get(nb + extra));
    GV_REQUIRE(base, "gv_accept_match: out of device memory");
    const Nuclei nu = carve(base, n, kMaxCand);
    int32_t *dbatch = reinterpret_cast<int32_t *>(base + nb);
    int32_t *dout = dbatch + 32;
    int *dres = reinterpret_cast<int *>(dout + 32);
    int32_t *dfresh = reinterpret_cast<int32_t *>(dres + 4);
    int32_t *dstop = dfresh + 33;
    int32_t *dseen = dstop + n_stop;
    const hipStream_t st = stream();
    GV_CHECK_HIP(hipMemcpyAsync(dbatch, batch, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, st));
    if (n_stop) GV_CHECK_HIP(hipMemcpyAsync(dstop, stop, static_cast<size_t>(n_stop) * 4, hipMemcpyHostToDevice, st));
    if (penalize) {
        GV_CHECK_HIP(hipMemcpyAsync(dfresh, fresh.data(), 33 * 4, hipMemcpyHostToDevice, st));
        if (n_seen) GV_CHECK_HIP(hipMemcpyAsync(dseen, seen, static_cast<size_t>(n_seen) * 4, hipMemcpyHostToDevice, st));
        hipLaunchKernelGGL(penalty_kernel, dim3(n), dim3(256), 0, st, logits, ld, dseen, n_seen, dbatch, dfresh,
                           presence_penalty);
        GV_CHECK_HIP(hipGetLastError());
    }
    if (nuclei(logits, ld, n, V, temperature, top_p, top_k, cap, u, nu, st) != 0) return -1;
    hipLaunchKernelGGL(match_kernel, dim3(1), dim3(64), 0, st, nu.pick, dbatch, n, dstop, n_stop, dout, dres);
    GV_CHECK_HIP(hipGetLastError());
    int res[2] = {0, 0};
    GV_CHECK_HIP(hipMemcpyAsync(res, dres, 8, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    GV_CHECK_HIP(hipMemcpy(out, dout, static_cast<size_t>(res[0]) * 4, hipMemcpyDeviceToHost));
    if (kept) *kept = res[1];
    return res[0];
}

int gv_accept_textbook(const float *target, const float *draft, int64_t ld, int V, int k, float temperature,
                       float top_p, int greedy, const float *u_draft, const float *u_acc, float u_res, int32_t *out) {
    if (ensure_init() != 0) return -1;
    GV_REQUIRE(target && draft && out && k >= 1 && k <= 31 && V >= 1 && ld >= V, "gv_accept_textbook: bad arguments");
    GV_REQUIRE(greedy || (u_draft && u_acc && temperature > 0.0f), "gv_accept_textbook: uniforms and T > 0 needed");
    const int R = 2 * k + 1;
    const size_t nb = nuclei_bytes(R, kMaxCand);
    const size_t qb = static_cast<size_t>(V) * 8;
    char *base = static_cast<char *>(ws().get(nb + qb + 1024));
    GV_REQUIRE(base, "gv_accept_textbook: out of device memory");
    double *qq = reinterpret_cast<double *>(base + nb);
    float *dacc = reinterpret_cast<float *>(base + nb + qb);
    int32_t *dout = reinterpret_cast<int32_t *>(dacc + 32);
    int *dres = reinterpret_cast<int *>(dout + 32);
    const hipStream_t st = stream();
    GV_CHECK_HIP(hipMemsetAsync(qq, 0, qb, st));
    // target rows 0..k (row k draws the bonus with u_res; rows < k draw nothing used), draft rows 0..k-1 (u_draft)
    std::vector<double> ut(static_cast<size_t>(k) + 1, 0.0), ud(static_cast<size_t>(k), 0.0);
    ut[static_cast<size_t>(k)] = u_res;
    for (int i = 0; i < k; ++i) {
        ut[static_cast<size_t>(i)] = u_res;   // a rejected row with no residual mass draws from p with u_res
        ud[static_cast<size_t>(i)] = greedy ? 0.0 : u_draft[i];
    }
    const float Tn = greedy ? 0.0f : temperature;
    const Nuclei np = carve(base, R, kMaxCand);
    Nuclei nq = np;   // draft rows after the k + 1 target rows
    nq.key += (k + 1) * np.cs;
    nq.idx += (k + 1) * np.cs;
    nq.e += (k + 1) * np.cs;
    nq.sum += k + 1;
    nq.kept += k + 1;
    nq.u += k + 1;
    nq.keep += k + 1;
    nq.pos += k + 1;
    nq.pick += k + 1;
    nq.flag = np.flag;
    if (nuclei(target, ld, k + 1, V, Tn, top_p, 0, 0, ut.data(), np, st) != 0) return -1;
    if (nuclei(draft, ld, k, V, Tn, top_p, 0, 0, ud.data(), nq, st) != 0) return -1;
    if (!greedy) GV_CHECK_HIP(hipMemcpyAsync(dacc, u_acc, static_cast<size_t>(k) * 4, hipMemcpyHostToDevice, st));
    static int granted = 0;
    const size_t lds = static_cast<size_t>(kMaxCand) * 8;
    if (lds_grant(reinterpret_cast<const void *>(&textbook_kernel), lds, granted) != 0) return -1;
    hipLaunchKernelGGL(textbook_kernel, dim3(1), dim3(kSelThreads), lds, st, np.rows(0), nq.rows(0), k, greedy, dacc,
                       u_res, qq, dout, dres);
    GV_CHECK_HIP(hipGetLastError());
    int res = 0;
    GV_CHECK_HIP(hipMemcpyAsync(&res, dres, 4, hipMemcpyDeviceToHost, st));
    GV_CHECK_HIP(hipStreamSynchronize(st));
    GV_CHECK_HIP(hipMemcpy(out, dout, static_cast<size_t>(res) * 4, hipMemcpyDeviceToHost));
    return res;
}

}  // extern "C"
