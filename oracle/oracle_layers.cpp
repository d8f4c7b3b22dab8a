// oracle_layers.cpp - the verify step's layers on the CPU: the dense SwiGLU MLP, the MoE block, gated attention with
// the causal chain or a draft tree, and the whole forward pass of a batch (verify_n / verify_keep).
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP path, never part of it.
//
// Pinning: the reference's Model does not build without a real pack, so these compositions are pinned
// (tests/test_oracle_layers.py) against an independent float64 restatement of the whole forward pass written from
// the reference's formulas (tests/f64_model.py: RMSNorm(1 + w), gated q, q/k norm, RoPE pairs (i, i + half), fp16
// KV, 1/sqrt(hd) softmax, sigmoid gate, bf16 router, renormalised top-K, SwiGLU experts, sigmoid-gated shared
// expert), in both arithmetic modes, chain and tree: logits within 4e-6 (exact path) and 4e-5 (int8 path), routing
// identical; eleven planted slips in the restatement (a dropped scale or gate, a RoPE sign or pairing, the norm's
// (1 + w), the renormalisation, silu, the mask, the fp16 KV rounding) each land far outside that. The MoE block
// alone against a dense float64 brute force (every expert computed, the unpicked ones weighted 0); attention bits
// independent of the block size up to the merge (model.cpp:3799-3855). tests/test_oracle_kv8.py adds the
// reference's stated invariants: verify logits equal one-token-at-a-time logits bit for bit (model.hpp:189-193), a
// tree row equals the chain over its ancestors, verify + keep equals a verify of the kept prefix.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <vector>

#include "oracle.h"
#include "oracle_internal.hpp"

namespace orc {

namespace {

std::vector<float *> row_ptrs(float *base, int n, size_t stride) {
    std::vector<float *> v(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) v[static_cast<size_t>(t)] = base + static_cast<size_t>(t) * stride;
    return v;
}
std::vector<const float *> crow_ptrs(const float *base, int n, size_t stride) {
    std::vector<const float *> v(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) v[static_cast<size_t>(t)] = base + static_cast<size_t>(t) * stride;
    return v;
}

// down(silu(gate h) * up h) for n tokens, gate and up separate matrices (the shared expert, model.cpp:4279-4296;
// the dense MLP, :4126-4146)
void swiglu_mlp(const uint8_t *gate, const uint8_t *up, const uint8_t *down, float gg, float gu, float gd, int H, int F,
                int n, const float *h, int mode, float *out) {
    std::vector<float> g(static_cast<size_t>(n) * F), u(static_cast<size_t>(n) * F);
    const auto hs = crow_ptrs(h, n, static_cast<size_t>(H));
    auto gs = row_ptrs(g.data(), n, static_cast<size_t>(F));
    auto us = row_ptrs(u.data(), n, static_cast<size_t>(F));
    matmul(gate, F, H, gg, n, hs.data(), gs.data(), mode);
    matmul(up, F, H, gu, n, hs.data(), us.data(), mode);
    for (size_t i = 0; i < g.size(); ++i) g[i] = silu(g[i]) * u[i];
    const auto ms = crow_ptrs(g.data(), n, static_cast<size_t>(F));
    auto os = row_ptrs(out, n, static_cast<size_t>(H));
    matmul(down, H, F, gd, n, ms.data(), os.data(), mode);
}

}  // namespace

// The MoE block of model.cpp:4123-4587 for n tokens (no residual). Each pick is computed whole, as one expert alone
// (every path of the reference gives these bits, model.cpp:4305-4308): gate_up h, silu(gate) * up, down.
void moe_layer(const orc_moe_weights &w, int n, const float *h, const float *router_logits, int mode, float *out,
               int *ids_out, float *wts_out, float *gate_out) {
    const int H = w.H, E = w.E, K = w.K, F = w.F;
    std::vector<float> logits(static_cast<size_t>(n) * E);
    if (router_logits) {
        std::copy(router_logits, router_logits + static_cast<size_t>(n) * E, logits.begin());
    } else {
        const auto hs = crow_ptrs(h, n, static_cast<size_t>(H));
        auto ls = row_ptrs(logits.data(), n, static_cast<size_t>(E));
        par(E, 16, [&](int64_t a, int64_t b) { bf16_rows(w.router, H, n, hs.data(), ls.data(), a, b); });
    }
    std::vector<int> ids(static_cast<size_t>(n) * K);
    std::vector<float> wts(static_cast<size_t>(n) * K);
    for (int t = 0; t < n; ++t)
        route_topk(logits.data() + static_cast<size_t>(t) * E, E, K, ids.data() + static_cast<size_t>(t) * K,
                   wts.data() + static_cast<size_t>(t) * K);
    const size_t gu_bytes = static_cast<size_t>(2 * F) * q4_row_bytes(H);
    const size_t blk_bytes = gu_bytes + static_cast<size_t>(H) * q4_row_bytes(F);
    std::vector<float> eout(static_cast<size_t>(n) * K * H);
    std::vector<float> ga(static_cast<size_t>(2 * F));
    for (int t = 0; t < n; ++t)
        for (int k = 0; k < K; ++k) {
            const int e = ids[static_cast<size_t>(t * K + k)];
            const uint8_t *blk = w.experts + static_cast<size_t>(e) * blk_bytes;
            const float *ht = h + static_cast<size_t>(t) * H;
            float *gp = ga.data();
            matmul(blk, 2 * F, H, w.expert_globals[2 * e], 1, &ht, &gp, mode);   // [gate F | up F]
            for (int i = 0; i < F; ++i) ga[static_cast<size_t>(i)] = silu(ga[static_cast<size_t>(i)]) * ga[static_cast<size_t>(F + i)];
            const float *mp = ga.data();
            float *yp = eout.data() + (static_cast<size_t>(t) * K + static_cast<size_t>(k)) * H;
            matmul(blk + gu_bytes, H, F, w.expert_globals[2 * e + 1], 1, &mp, &yp, mode);
        }
    std::vector<float> sh(static_cast<size_t>(n) * H);
    swiglu_mlp(w.sh_gate, w.sh_up, w.sh_down, w.sh_globals[0], w.sh_globals[1], w.sh_globals[2], H, w.SF, n, h, mode,
               sh.data());
    // per token: sigmoid(bf16 gate . h) times the shared expert, then the routed outputs in rank order
    for (int t = 0; t < n; ++t) {
        const float *ht = h + static_cast<size_t>(t) * H;
        float gs = 0.0f;
        for (int i = 0; i < H; ++i) gs += bf16_to_f32(w.shared_gate[i]) * ht[i];
        gs = sigmoid(gs);
        if (gate_out) gate_out[t] = gs;
        float *o = out + static_cast<size_t>(t) * H;
        const float *shv = sh.data() + static_cast<size_t>(t) * H;
        for (int i = 0; i < H; ++i) o[i] = gs * shv[i];
        for (int k = 0; k < K; ++k) {
            const float wk = wts[static_cast<size_t>(t * K + k)];
            if (wk == 0.0f) continue;
            const float *y = eout.data() + (static_cast<size_t>(t) * K + static_cast<size_t>(k)) * H;
            for (int i = 0; i < H; ++i) o[i] += wk * y[i];
        }
    }
    if (ids_out) std::copy(ids.begin(), ids.end(), ids_out);
    if (wts_out) std::copy(wts.begin(), wts.end(), wts_out);
}

// ---------------------------------------------------------------- Gated DeltaNet (model.cpp:3497-3688)
// fast_exp (kernels.hpp:142-163): Cephes' expf (the reduction by ln 2 in two parts, a degree-6 polynomial, 2^n by
// the exponent's bits), within 2 ulp; below -87 it is e^-87
float fast_exp(float x) {
    x = std::fmin(std::fmax(x, -87.0f), 88.0f);
    const float n = std::floor(x * 1.44269504088896341f + 0.5f);
    float r = x - n * 0.693359375f;
    r = r + n * 2.12194440e-4f;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = p * r * r + r + 1.0f;
    uint32_t bits;
    std::memcpy(&bits, &p, 4);
    bits += static_cast<uint32_t>(static_cast<int32_t>(n)) << 23;
    std::memcpy(&p, &bits, 4);
    return p;
}
float silu_fast(float x) { return x / (1.0f + fast_exp(-x)); }   // kernels.hpp:165
float softplus(float x) { return x > 20.0f ? x : std::log1p(std::exp(x)); }   // kernels.hpp:168

// one token of the delta rule on one head's state S [dk][dv] (the generic loop of model.cpp:3602-3627): column j
// sums over the rows in order
void delta_step(float *S, int dk, int dv, const float *q, const float *k, const float *v, float decay, float beta,
                float *out) {
    std::vector<float> mem(static_cast<size_t>(dv), 0.0f), o(static_cast<size_t>(dv), 0.0f);
    for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) {
            S[i * dv + j] *= decay;
            mem[static_cast<size_t>(j)] += S[i * dv + j] * k[i];
        }
    for (int j = 0; j < dv; ++j) mem[static_cast<size_t>(j)] = (v[j] - mem[static_cast<size_t>(j)]) * beta;
    for (int i = 0; i < dk; ++i)
        for (int j = 0; j < dv; ++j) {
            S[i * dv + j] += k[i] * mem[static_cast<size_t>(j)];
            o[static_cast<size_t>(j)] += S[i * dv + j] * q[i];
        }
    std::copy(o.begin(), o.end(), out);
}

// ---------------------------------------------------------------- the model
struct Layer {
    std::vector<float> in_norm, post_norm, q_norm, k_norm;
    std::vector<uint8_t> q, k, v, o, experts, sh_gate, sh_up, sh_down;
    float gq = 1, gk = 1, gv = 1, go = 1, gsg = 1, gsu = 1, gsd = 1;
    std::vector<float> expert_globals;   // [E][2]
    std::vector<uint16_t> router, shared_gate, kv;   // kv: [2][max_ctx][nkv * hd] fp16
    std::vector<int8_t> kv8;                         // int8 KV: [2][max_ctx][nkv * hd]
    std::vector<float> kvs;                          // int8 KV: [2][max_ctx][nkv] scales
    // a Gated DeltaNet layer (model.cpp:129-138) instead of the attention
    bool gdn = false;
    std::vector<uint8_t> gqkv, gz, gout;             // q4 [2 kd + vd][H], [vd][H], [H][vd]
    float g_qkv = 1, g_z = 1, g_out = 1;
    std::vector<uint16_t> ga, gb;                    // bf16 [nv][H]
    std::vector<float> A_log, dt_bias, conv_w, gnorm;   // [nv], [nv], [2 kd + vd][K], [dv]
    std::vector<float> conv_st, S;                   // [2 kd + vd][K - 1], [nv][dk][dv]
    std::vector<float> conv_bk, S_bk;                // the last verify's rows' states (verify_keep takes them back)
};

}  // namespace orc

struct orc_model {
    orc_config c{};
    std::vector<uint8_t> embed, lm_head;
    float g_embed = 1, g_lm = 1;
    std::vector<float> final_norm, inv_freq;
    std::vector<orc::Layer> layers;   // [n_layers] (+ the MTP layer's, index n_layers)
    int pos = 0, last_n = 0, last_pos = 0;
    // the MTP layer's own tensors (model.cpp:178-190)
    std::vector<uint8_t> mtp_fc;   // q4 [H][2 H]
    float g_fc = 1;
    std::vector<float> mtp_norm, mtp_pre_e, mtp_pre_h;
    std::vector<float> hid;        // the last verify's final-normed rows [last_n][H] (the MTP layer's input)
    std::vector<int> hid_rows;     // after a keep with a path: the kept rows (row t of a draft: hid row hid_rows[t])
    std::vector<float> mtp_out;    // the last MTP pass's last row after mtp.norm (draft_next's hidden state)
    std::vector<int32_t> draft_ids;     // the draft vocabulary (empty: the whole vocabulary)
    std::vector<uint8_t> draft_head;    // lm_head's rows of draft_ids
    double t_layers = 0, t_head = 0;
};

namespace orc {
namespace {

size_t expert_block_bytes(const orc_config &c) {   // pack.cpp:329-333
    return static_cast<size_t>(2 * c.moe_ff) * q4_row_bytes(c.hidden) +
           static_cast<size_t>(c.hidden) * q4_row_bytes(c.moe_ff);
}

// depth of each row of a draft tree (chain when parents is null)
std::vector<int> depths(const int32_t *parents, int n) {
    std::vector<int> d(static_cast<size_t>(n), 0);
    for (int i = 0; i < n; ++i) d[static_cast<size_t>(i)] = parents ? (parents[i] < 0 ? 0 : d[static_cast<size_t>(parents[i])] + 1) : i;
    return d;
}

// visible[i][j]: row j is row i or one of its ancestors (chain: j <= i)
std::vector<char> ancestry(const int32_t *parents, int n) {
    std::vector<char> a(static_cast<size_t>(n) * n, 0);
    for (int i = 0; i < n; ++i) {
        if (!parents) {
            for (int j = 0; j <= i; ++j) a[static_cast<size_t>(i) * n + j] = 1;
            continue;
        }
        for (int j = i; j >= 0; j = parents[j]) a[static_cast<size_t>(i) * n + j] = 1;
    }
    return a;
}

// quant_kv_row (model.cpp:3766-3774)
void quant_kv_row(const float *x, int n, int8_t *q, float &scale) {
    float amax = 0.0f;
    for (int i = 0; i < n; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    for (int i = 0; i < n; ++i) q[i] = static_cast<int8_t>(std::clamp(std::nearbyint(x[i] * inv), -127.0f, 127.0f));
    scale = amax / 127.0f;
}

// Model::attention + attend + attend_heads (model.cpp:3690-4019) for the n rows at slots pos.., rotary positions
// pos + depth. KV in fp16 (attend<_Float16>) or int8 (attend<int8_t>: a scale a position and KV head, the K scale
// in the score's factor, model.cpp:3929-3948, the V scale in the weights after their sum, :3965-3972). h: the
// in-norm's output; mix: o_proj's.
void attention(const orc_model &m, Layer &L, int n, const float *h, int pos, const int32_t *parents, int mode,
               float *mix) {
    const auto &c = m.c;
    const int H = c.hidden, nh = c.n_heads, nkv = c.n_kv_heads, hd = c.head_dim, half = c.rope_dim / 2;
    const size_t kv_row = static_cast<size_t>(nkv) * hd, qw = static_cast<size_t>(nh) * 2 * hd;
    std::vector<float> qs(static_cast<size_t>(n) * qw), ks(static_cast<size_t>(n) * kv_row),
        vs(static_cast<size_t>(n) * kv_row);
    const auto hs = crow_ptrs(h, n, static_cast<size_t>(H));
    {
        auto qp = row_ptrs(qs.data(), n, qw);
        auto kp = row_ptrs(ks.data(), n, kv_row);
        auto vp = row_ptrs(vs.data(), n, kv_row);
        matmul(L.q.data(), static_cast<int64_t>(qw), H, L.gq, n, hs.data(), qp.data(), mode);
        matmul(L.k.data(), static_cast<int64_t>(kv_row), H, L.gk, n, hs.data(), kp.data(), mode);
        matmul(L.v.data(), static_cast<int64_t>(kv_row), H, L.gv, n, hs.data(), vp.data(), mode);
    }
    const std::vector<int> dep = depths(parents, n);
    std::vector<float> cosv(static_cast<size_t>(half)), sinv(static_cast<size_t>(half));
    auto rope = [&](float *x) {
        for (int i = 0; i < half; ++i) {
            const float x1 = x[i], x2 = x[i + half];
            x[i] = x1 * cosv[static_cast<size_t>(i)] - x2 * sinv[static_cast<size_t>(i)];
            x[i + half] = x2 * cosv[static_cast<size_t>(i)] + x1 * sinv[static_cast<size_t>(i)];
        }
    };
    for (int t = 0; t < n; ++t) {
        const int p = pos + dep[static_cast<size_t>(t)];   // text: the three M-RoPE streams are one (model.cpp:1746-1760)
        for (int i = 0; i < half; ++i) {
            const float f = static_cast<float>(p) * m.inv_freq[static_cast<size_t>(i)];
            cosv[static_cast<size_t>(i)] = std::cos(f);
            sinv[static_cast<size_t>(i)] = std::sin(f);
        }
        for (int hh = 0; hh < nh; ++hh) {
            float *q = qs.data() + static_cast<size_t>(t) * qw + static_cast<size_t>(hh) * 2 * hd;
            rmsnorm(q, L.q_norm.data(), q, hd, c.eps, true);
            rope(q);
        }
        for (int kh = 0; kh < nkv; ++kh) {
            float *k = ks.data() + static_cast<size_t>(t) * kv_row + static_cast<size_t>(kh) * hd;
            rmsnorm(k, L.k_norm.data(), k, hd, c.eps, true);
            rope(k);
        }
    }
    const bool i8 = c.kv_int8 != 0;
    uint16_t *K = i8 ? nullptr : L.kv.data(), *V = i8 ? nullptr : L.kv.data() + static_cast<size_t>(c.max_ctx) * kv_row;
    int8_t *K8 = i8 ? L.kv8.data() : nullptr, *V8 = i8 ? L.kv8.data() + static_cast<size_t>(c.max_ctx) * kv_row : nullptr;
    float *KS = i8 ? L.kvs.data() : nullptr, *VS = i8 ? L.kvs.data() + static_cast<size_t>(c.max_ctx) * nkv : nullptr;
    for (int t = 0; t < n; ++t) {
        if (i8) {   // attend<int8_t> (model.cpp:3787-3792)
            for (int kh = 0; kh < nkv; ++kh) {
                const size_t o = static_cast<size_t>(kh) * hd, r = static_cast<size_t>(pos + t);
                quant_kv_row(ks.data() + static_cast<size_t>(t) * kv_row + o, hd, K8 + r * kv_row + o, KS[r * nkv + kh]);
                quant_kv_row(vs.data() + static_cast<size_t>(t) * kv_row + o, hd, V8 + r * kv_row + o, VS[r * nkv + kh]);
            }
            continue;
        }
        for (size_t i = 0; i < kv_row; ++i) {
            K[static_cast<size_t>(pos + t) * kv_row + i] = f32_to_f16(ks[static_cast<size_t>(t) * kv_row + i]);
            V[static_cast<size_t>(pos + t) * kv_row + i] = f32_to_f16(vs[static_cast<size_t>(t) * kv_row + i]);
        }
    }
    auto kval = [&](int s, int kh, int i) {   // K as the attention reads it: fp16, or the int8 value itself
        const size_t o = static_cast<size_t>(s) * kv_row + static_cast<size_t>(kh) * hd + i;
        return i8 ? static_cast<float>(K8[o]) : f16_to_f32(K[o]);
    };
    auto vval = [&](int s, int kh, int i) {
        const size_t o = static_cast<size_t>(s) * kv_row + static_cast<size_t>(kh) * hd + i;
        return i8 ? static_cast<float>(V8[o]) : f16_to_f32(V[o]);
    };
    const std::vector<char> vis = ancestry(parents, n);
    const int group = nh / nkv, blk = c.attn_block;
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    std::vector<float> core(static_cast<size_t>(n) * nh * hd);
    par(static_cast<int64_t>(n) * nh, 1, [&](int64_t i0, int64_t i1) {
        std::vector<float> sc, part, o(static_cast<size_t>(hd));
        std::vector<int> slots;
        for (int64_t it = i0; it < i1; ++it) {
            const int t = static_cast<int>(it / nh), hh = static_cast<int>(it % nh), kh = hh / group;
            const float *q = qs.data() + static_cast<size_t>(t) * qw + static_cast<size_t>(hh) * 2 * hd;
            const float *gate = q + hd;
            const int last = pos + t;
            const int nb = last / blk + 1;
            part.assign(static_cast<size_t>(nb) * (hd + 2), 0.0f);
            for (int b = 0; b < nb; ++b) {
                slots.clear();
                for (int s = b * blk; s < std::min(last + 1, (b + 1) * blk); ++s)
                    if (s < pos || vis[static_cast<size_t>(t) * n + (s - pos)]) slots.push_back(s);
                float mx = -std::numeric_limits<float>::infinity();
                sc.resize(slots.size());
                for (size_t p = 0; p < slots.size(); ++p) {
                    float acc[8] = {};
                    for (int i = 0; i < hd; i += 8)
                        for (int j = 0; j < 8; ++j) acc[j] += q[i + j] * kval(slots[p], kh, i + j);
                    const float dot = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
                    const float f = i8 ? scale * KS[static_cast<size_t>(slots[p]) * nkv + kh] : scale;
                    const float sv = dot * f;
                    sc[p] = sv;
                    mx = std::max(mx, sv);
                }
                float sum = 0.0f;
                for (size_t p = 0; p < slots.size(); ++p) {
                    sc[p] = std::exp(sc[p] - mx);
                    sum += sc[p];
                }
                if (i8)   // each position's V scale into its weights (the sum above is the softmax's own)
                    for (size_t p = 0; p < slots.size(); ++p) sc[p] *= VS[static_cast<size_t>(slots[p]) * nkv + kh];
                float *dst = part.data() + static_cast<size_t>(b) * (hd + 2);
                dst[hd] = mx;
                dst[hd + 1] = sum;
                for (int i = 0; i < hd; i += 8) {
                    float acc[8] = {};
                    for (size_t p = 0; p < slots.size(); ++p)
                        for (int j = 0; j < 8; ++j) acc[j] += sc[p] * vval(slots[p], kh, i + j);
                    std::memcpy(dst + i, acc, sizeof acc);
                }
            }
            float sum = part[static_cast<size_t>(hd) + 1];
            if (nb == 1) {
                std::copy(part.begin(), part.begin() + hd, o.begin());
            } else {
                float mx = -std::numeric_limits<float>::infinity();
                for (int b = 0; b < nb; ++b) mx = std::max(mx, part[static_cast<size_t>(b) * (hd + 2) + hd]);
                std::fill(o.begin(), o.end(), 0.0f);
                sum = 0.0f;
                for (int b = 0; b < nb; ++b) {
                    const float *pp = part.data() + static_cast<size_t>(b) * (hd + 2);
                    const float f = std::exp(pp[hd] - mx);
                    sum += pp[hd + 1] * f;
                    for (int j = 0; j < hd; ++j) o[static_cast<size_t>(j)] += pp[j] * f;
                }
            }
            const float inv = 1.0f / sum;
            float *out = core.data() + (static_cast<size_t>(t) * nh + hh) * hd;
            for (int j = 0; j < hd; ++j) out[j] = o[static_cast<size_t>(j)] * inv * sigmoid(gate[j]);
        }
    });
    const auto cr = crow_ptrs(core.data(), n, static_cast<size_t>(nh) * hd);
    auto ms = row_ptrs(mix, n, static_cast<size_t>(H));
    matmul(L.o.data(), H, static_cast<int64_t>(nh) * hd, L.go, n, cr.data(), ms.data(), mode);
}

orc_moe_weights moe_view(const orc_model &m, const Layer &L) {
    orc_moe_weights w{};
    w.H = m.c.hidden, w.E = m.c.n_experts, w.K = m.c.top_k, w.F = m.c.moe_ff, w.SF = m.c.shared_ff;
    w.experts = L.experts.data();
    w.expert_globals = L.expert_globals.data();
    w.sh_gate = L.sh_gate.data(), w.sh_up = L.sh_up.data(), w.sh_down = L.sh_down.data();
    w.sh_globals[0] = L.gsg, w.sh_globals[1] = L.gsu, w.sh_globals[2] = L.gsd;
    w.shared_gate = L.shared_gate.data();
    w.router = L.router.data();
    return w;
}

// A Gated DeltaNet layer on n rows h (model.cpp:3526-3688): the projections (the int8 path in mode 0, model.cpp:
// 3540-3547), the bf16 a / b rows, the causal conv over the last K inputs + silu (:3558-3584), q and k L2-normalised
// per key head, q by 1/sqrt(dk) (:3586-3603), beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias))
// (:3605-3612), the delta rule per value head (:3614-3666), the gated RMSNorm o / rms(o) w silu(z) (:3670-3682), the
// output projection into mix. A row's states start from its parent's (parents null: the row before; the first row:
// the layer's), and every row's states are kept (conv_bk, S_bk): a chain ends with its last row's in the layer,
// verify_keep takes back those of the last kept row.
void gdn_layer(const orc_model &m, Layer &L, int n, const float *h, const int32_t *parents, int mode, float *mix) {
    const auto &c = m.c;
    const int H = c.hidden, nk = c.gdn_k_heads, nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim, K = c.conv_kernel;
    const int kd = nk * dk, vd = nv * dv, conv_dim = 2 * kd + vd, rep = nv / nk;
    const size_t cs_n = static_cast<size_t>(conv_dim) * (K - 1), s_n = static_cast<size_t>(nv) * dk * dv;
    std::vector<float> proj(static_cast<size_t>(n) * conv_dim), z(static_cast<size_t>(n) * vd), a(static_cast<size_t>(n) * nv),
        b(static_cast<size_t>(n) * nv), core(static_cast<size_t>(n) * vd);
    const auto hs = crow_ptrs(h, n, static_cast<size_t>(H));
    {
        auto ps = row_ptrs(proj.data(), n, static_cast<size_t>(conv_dim));
        auto zs = row_ptrs(z.data(), n, static_cast<size_t>(vd));
        matmul(L.gqkv.data(), conv_dim, H, L.g_qkv, n, hs.data(), ps.data(), mode);
        matmul(L.gz.data(), vd, H, L.g_z, n, hs.data(), zs.data(), mode);
        auto as = row_ptrs(a.data(), n, static_cast<size_t>(nv));
        auto bs = row_ptrs(b.data(), n, static_cast<size_t>(nv));
        bf16_rows(L.ga.data(), H, n, hs.data(), as.data(), 0, nv);
        bf16_rows(L.gb.data(), H, n, hs.data(), bs.data(), 0, nv);
    }
    L.conv_bk.assign(static_cast<size_t>(n) * cs_n, 0.0f);
    L.S_bk.assign(static_cast<size_t>(n) * s_n, 0.0f);
    const float qscale = 1.0f / std::sqrt(static_cast<float>(dk));
    for (int t = 0; t < n; ++t) {
        const int parent = parents ? parents[t] : t - 1;
        // the conv: the parent's last K - 1 inputs, then this row's; the new state is the last K - 1 of them
        const float *cin = parent < 0 ? L.conv_st.data() : L.conv_bk.data() + static_cast<size_t>(parent) * cs_n;
        float *cout = L.conv_bk.data() + static_cast<size_t>(t) * cs_n;
        float *row = proj.data() + static_cast<size_t>(t) * conv_dim;
        for (int ch = 0; ch < conv_dim; ++ch) {
            const float *w = L.conv_w.data() + static_cast<size_t>(ch) * K;
            const float *st = cin + static_cast<size_t>(ch) * (K - 1);
            float *so = cout + static_cast<size_t>(ch) * (K - 1);
            const float in = row[ch];
            float acc = 0.0f;
            for (int k = 0; k < K - 1; ++k) acc += w[k] * st[k];
            acc += w[K - 1] * in;
            for (int k = 0; k + 1 < K - 1; ++k) so[k] = st[k + 1];
            if (K > 1) so[K - 2] = in;
            row[ch] = silu_fast(acc);
        }
        for (int kh = 0; kh < nk; ++kh) {   // q, k: L2-normalised, q scaled
            float *q = row + kh * dk, *k = row + kd + kh * dk;
            float sq = 0.0f, sk = 0.0f;
            for (int j = 0; j < dk; ++j) {
                sq += q[j] * q[j];
                sk += k[j] * k[j];
            }
            const float iq = 1.0f / std::sqrt(sq + 1e-6f), ik = 1.0f / std::sqrt(sk + 1e-6f);
            for (int j = 0; j < dk; ++j) {
                q[j] = q[j] * iq * qscale;
                k[j] = k[j] * ik;
            }
        }
        const float *sin = parent < 0 ? L.S.data() : L.S_bk.data() + static_cast<size_t>(parent) * s_n;
        float *sout = L.S_bk.data() + static_cast<size_t>(t) * s_n;
        std::copy(sin, sin + s_n, sout);
        for (int vh = 0; vh < nv; ++vh) {
            const int kh = vh / rep;
            const float beta = sigmoid(b[static_cast<size_t>(t) * nv + vh]);
            const float decay = std::exp(-std::exp(L.A_log[static_cast<size_t>(vh)]) *
                                         softplus(a[static_cast<size_t>(t) * nv + vh] + L.dt_bias[static_cast<size_t>(vh)]));
            float *o = core.data() + static_cast<size_t>(t) * vd + static_cast<size_t>(vh) * dv;
            delta_step(sout + static_cast<size_t>(vh) * dk * dv, dk, dv, row + kh * dk, row + kd + kh * dk,
                       row + 2 * kd + vh * dv, decay, beta, o);
            float ss = 0.0f;   // the gated RMSNorm of the head's output
            for (int j = 0; j < dv; ++j) ss += o[j] * o[j];
            const float inv = 1.0f / std::sqrt(ss / static_cast<float>(dv) + c.eps);
            const float *zz = z.data() + static_cast<size_t>(t) * vd + static_cast<size_t>(vh) * dv;
            for (int j = 0; j < dv; ++j) o[j] = o[j] * inv * L.gnorm[static_cast<size_t>(j)] * silu_fast(zz[j]);
        }
    }
    // (the chain's end: the last row's states; a tree's keep takes back the right ones)
    std::copy(L.conv_bk.end() - static_cast<ptrdiff_t>(cs_n), L.conv_bk.end(), L.conv_st.begin());
    std::copy(L.S_bk.end() - static_cast<ptrdiff_t>(s_n), L.S_bk.end(), L.S.begin());
    const auto cr = crow_ptrs(core.data(), n, static_cast<size_t>(vd));
    auto ms = row_ptrs(mix, n, static_cast<size_t>(H));
    matmul(L.gout.data(), H, vd, L.g_out, n, cr.data(), ms.data(), mode);
}

uint64_t tensor_seed(uint64_t seed, int kind, int layer, int expert) {
    return orc_hash(seed, (static_cast<uint64_t>(kind) << 48) | (static_cast<uint64_t>(layer) << 24) |
                              static_cast<uint64_t>(expert));
}

float fill_q4(std::vector<uint8_t> &dst, int64_t rows, int64_t cols, uint64_t seed, float sigma, int fast) {
    dst.resize(static_cast<size_t>(rows) * q4_row_bytes(cols));
    if (fast) {
        const int64_t nb = cols / 16;
        const size_t rb = q4_row_bytes(cols);
        // (eight code bytes a hash; each scale byte from a byte of a hash: 0x30 + b % 25, exponents 6..9)
        par(rows, 64, [&](int64_t a, int64_t b) {
            for (int64_t r = a; r < b; ++r) {
                uint8_t *row = dst.data() + static_cast<size_t>(r) * rb;
                for (int64_t i = 0; i < nb; ++i) {
                    const uint64_t h = orc_hash(seed, static_cast<uint64_t>(r * nb + i));
                    std::memcpy(row + 8 * i, &h, 8);
                    row[nb * 8 + i] = static_cast<uint8_t>(0x30 + ((orc_hash(seed ^ 1, static_cast<uint64_t>(r * nb + i)) >> 24) & 0xFF) % 25);
                }
            }
        });
        return 1.0f / 448.0f;
    }
    std::vector<float> w(static_cast<size_t>(rows) * cols);
    orc_fill_normal(seed, static_cast<int64_t>(w.size()), 0.0f, sigma, w.data());
    const float s2 = orc_q4_global(w.data(), static_cast<int64_t>(w.size()));
    orc_q4_pack(w.data(), rows, cols, s2, dst.data());
    return s2;
}

void fill_f32(std::vector<float> &dst, size_t n, uint64_t seed, float sigma) {
    dst.resize(n);
    orc_fill_normal(seed, static_cast<int64_t>(n), 0.0f, sigma, dst.data());
}

void fill_bf16(std::vector<uint16_t> &dst, size_t n, uint64_t seed, float sigma) {
    std::vector<float> f(n);
    orc_fill_normal(seed, static_cast<int64_t>(n), 0.0f, sigma, f.data());
    dst.resize(n);
    for (size_t i = 0; i < n; ++i) dst[i] = f32_to_bf16(f[i]);
}

}  // namespace
}  // namespace orc

using namespace orc;

extern "C" {

void orc_ffn_swiglu(const uint8_t *gate, const uint8_t *up, const uint8_t *down, float g_gate, float g_up,
                    float g_down, int H, int F, int M, const uint16_t *x_f16, int mode, float *y) {
    std::vector<float> x(static_cast<size_t>(M) * H);
    for (size_t i = 0; i < x.size(); ++i) x[i] = f16_to_f32(x_f16[i]);
    swiglu_mlp(gate, up, down, g_gate, g_up, g_down, H, F, M, x.data(), mode, y);
}

void orc_moe_layer(const orc_moe_weights *w, int M, const float *h, const float *router_logits, int mode, float *out,
                   int *ids, float *wts, float *gate) {
    moe_layer(*w, M, h, router_logits, mode, out, ids, wts, gate);
}

orc_model *orc_model_create(const orc_config *cfg) {
    auto m = std::make_unique<orc_model>();
    m->c = *cfg;
    if (m->c.attn_block <= 0) m->c.attn_block = 1024;
    const auto &c = m->c;
    const int half = c.rope_dim / 2;
    m->inv_freq.resize(static_cast<size_t>(half));
    for (int i = 0; i < half; ++i)   // model.cpp:739-740
        m->inv_freq[static_cast<size_t>(i)] =
            1.0f / std::pow(c.rope_theta, static_cast<float>(2 * i) / static_cast<float>(c.rope_dim));
    m->layers.resize(static_cast<size_t>(c.n_layers + (c.mtp ? 1 : 0)));
    return m.release();
}

void orc_model_free(orc_model *m) { delete m; }

float orc_fast_exp(float x) { return orc::fast_exp(x); }

void orc_gdn_step(float *S, int dk, int dv, const float *q, const float *k, const float *v, float decay, float beta,
                  float *out) {
    orc::delta_step(S, dk, dv, q, k, v, decay, beta, out);
}

void orc_quant_kv_row(const float *x, int n, int8_t *q, float *scale) { orc::quant_kv_row(x, n, q, *scale); }

void orc_model_fill(orc_model *m, uint64_t seed, float sigma, float router_sigma, int ctx, int fast) {
    const auto &c = m->c;
    const int H = c.hidden, E = c.n_experts, F = c.moe_ff, SF = c.shared_ff, nh = c.n_heads, nkv = c.n_kv_heads,
              hd = c.head_dim;
    m->g_embed = fill_q4(m->embed, c.vocab, H, tensor_seed(seed, ORC_EMBED, 0, 0), sigma, fast);
    m->g_lm = fill_q4(m->lm_head, c.vocab, H, tensor_seed(seed, ORC_LM_HEAD, 0, 0), sigma, fast);
    fill_f32(m->final_norm, static_cast<size_t>(H), tensor_seed(seed, ORC_FINAL_NORM, 0, 0), 0.02f);
    const size_t kv_row = static_cast<size_t>(nkv) * hd;
    if (c.mtp) {   // the MTP layer's fc and norms; its decoder layer is filled as layer n_layers below
        m->g_fc = fill_q4(m->mtp_fc, H, 2 * static_cast<int64_t>(H), tensor_seed(seed, ORC_MTP_FC, 0, 0), sigma, fast);
        fill_f32(m->mtp_norm, static_cast<size_t>(H), tensor_seed(seed, ORC_MTP_NORM, 0, 0), 0.02f);
        fill_f32(m->mtp_pre_e, static_cast<size_t>(H), tensor_seed(seed, ORC_MTP_PRE_E, 0, 0), 0.02f);
        fill_f32(m->mtp_pre_h, static_cast<size_t>(H), tensor_seed(seed, ORC_MTP_PRE_H, 0, 0), 0.02f);
    }
    for (int l = 0; l < static_cast<int>(m->layers.size()); ++l) {
        Layer &L = m->layers[static_cast<size_t>(l)];
        fill_f32(L.in_norm, static_cast<size_t>(H), tensor_seed(seed, ORC_IN_NORM, l, 0), 0.02f);
        fill_f32(L.post_norm, static_cast<size_t>(H), tensor_seed(seed, ORC_POST_NORM, l, 0), 0.02f);
        fill_f32(L.q_norm, static_cast<size_t>(hd), tensor_seed(seed, ORC_Q_NORM, l, 0), 0.02f);
        fill_f32(L.k_norm, static_cast<size_t>(hd), tensor_seed(seed, ORC_K_NORM, l, 0), 0.02f);
        L.gq = fill_q4(L.q, static_cast<int64_t>(nh) * 2 * hd, H, tensor_seed(seed, ORC_Q, l, 0), sigma, fast);
        L.gk = fill_q4(L.k, static_cast<int64_t>(kv_row), H, tensor_seed(seed, ORC_K, l, 0), sigma, fast);
        L.gv = fill_q4(L.v, static_cast<int64_t>(kv_row), H, tensor_seed(seed, ORC_V, l, 0), sigma, fast);
        L.go = fill_q4(L.o, H, static_cast<int64_t>(nh) * hd, tensor_seed(seed, ORC_O, l, 0), sigma, fast);
        fill_bf16(L.router, static_cast<size_t>(E) * H, tensor_seed(seed, ORC_ROUTER, l, 0), router_sigma);
        fill_bf16(L.shared_gate, static_cast<size_t>(H), tensor_seed(seed, ORC_SHARED_GATE, l, 0), sigma);
        const size_t eb = expert_block_bytes(c), gu = static_cast<size_t>(2 * F) * q4_row_bytes(H);
        L.experts.resize(eb * static_cast<size_t>(E));
        L.expert_globals.resize(static_cast<size_t>(2 * E));
        par(E, 1, [&](int64_t e0, int64_t e1) {   // experts on the pool's threads (each fill then runs in its thread)
            std::vector<uint8_t> tmp;
            for (int64_t e = e0; e < e1; ++e) {
                L.expert_globals[static_cast<size_t>(2 * e)] =
                    fill_q4(tmp, 2 * F, H, tensor_seed(seed, ORC_EXPERT, l, static_cast<int>(2 * e)), sigma, fast);
                std::copy(tmp.begin(), tmp.end(), L.experts.begin() + static_cast<ptrdiff_t>(eb * e));
                L.expert_globals[static_cast<size_t>(2 * e + 1)] =
                    fill_q4(tmp, H, F, tensor_seed(seed, ORC_EXPERT, l, static_cast<int>(2 * e + 1)), sigma, fast);
                std::copy(tmp.begin(), tmp.end(), L.experts.begin() + static_cast<ptrdiff_t>(eb * e + gu));
            }
        });
        L.gdn = c.gdn_v_heads > 0 && l < c.n_layers && c.gdn_layers[l] != 0;
        if (L.gdn) {   // the GDN layer's weights, then (a context) its states
            const int nk = c.gdn_k_heads, nv = c.gdn_v_heads, dk = c.gdn_k_dim, dv = c.gdn_v_dim, K = c.conv_kernel;
            const int kd = nk * dk, vd = nv * dv, conv_dim = 2 * kd + vd;
            L.g_qkv = fill_q4(L.gqkv, conv_dim, H, tensor_seed(seed, ORC_GDN_QKV, l, 0), sigma, fast);
            L.g_z = fill_q4(L.gz, vd, H, tensor_seed(seed, ORC_GDN_Z, l, 0), sigma, fast);
            L.g_out = fill_q4(L.gout, H, vd, tensor_seed(seed, ORC_GDN_OUT, l, 0), sigma, fast);
            fill_bf16(L.ga, static_cast<size_t>(nv) * H, tensor_seed(seed, ORC_GDN_A, l, 0), router_sigma);
            fill_bf16(L.gb, static_cast<size_t>(nv) * H, tensor_seed(seed, ORC_GDN_B, l, 0), router_sigma);
            fill_f32(L.A_log, static_cast<size_t>(nv), tensor_seed(seed, ORC_GDN_ALOG, l, 0), 0.5f);
            fill_f32(L.dt_bias, static_cast<size_t>(nv), tensor_seed(seed, ORC_GDN_DTB, l, 0), 0.5f);
            fill_f32(L.conv_w, static_cast<size_t>(conv_dim) * K, tensor_seed(seed, ORC_GDN_CONV, l, 0), 0.3f);
            fill_f32(L.gnorm, static_cast<size_t>(dv), tensor_seed(seed, ORC_GDN_NORM, l, 0), 0.02f);
            for (float &g : L.gnorm) g += 1.0f;
            L.conv_st.assign(static_cast<size_t>(conv_dim) * (K - 1), 0.0f);
            L.S.assign(static_cast<size_t>(nv) * dk * dv, 0.0f);
            if (ctx > 0) {   // a conversation's states: the conv's last inputs N(0, 1), the recurrent state N(0, 0.05)
                fill_f32(L.conv_st, L.conv_st.size(), tensor_seed(seed, ORC_GDN_CONV_ST, l, 0), 1.0f);
                fill_f32(L.S, L.S.size(), tensor_seed(seed, ORC_GDN_S, l, 0), 0.05f);
            }
        }
        L.gsg = fill_q4(L.sh_gate, SF, H, tensor_seed(seed, ORC_SH_GATE, l, 0), sigma, fast);
        L.gsu = fill_q4(L.sh_up, SF, H, tensor_seed(seed, ORC_SH_UP, l, 0), sigma, fast);
        L.gsd = fill_q4(L.sh_down, H, SF, tensor_seed(seed, ORC_SH_DOWN, l, 0), sigma, fast);
        if (c.kv_int8) {
            L.kv.clear();
            L.kv8.assign(2 * static_cast<size_t>(c.max_ctx) * kv_row, 0);
            L.kvs.assign(2 * static_cast<size_t>(c.max_ctx) * nkv, 0.0f);
        } else {
            L.kv.assign(2 * static_cast<size_t>(c.max_ctx) * kv_row, 0);
        }
        if (ctx > 0) {   // the context's keys and values N(0, 1), stored as the cache stores them
            std::vector<float> f(static_cast<size_t>(ctx) * kv_row);
            for (int kvi = 0; kvi < 2; ++kvi) {
                orc_fill_normal(tensor_seed(seed, ORC_KV, l, kvi), static_cast<int64_t>(f.size()), 0.0f, 1.0f, f.data());
                if (c.kv_int8) {
                    int8_t *dst = L.kv8.data() + static_cast<size_t>(kvi) * c.max_ctx * kv_row;
                    float *sd = L.kvs.data() + static_cast<size_t>(kvi) * c.max_ctx * nkv;
                    for (int p = 0; p < ctx; ++p)
                        for (int kh = 0; kh < nkv; ++kh) {
                            const size_t o = static_cast<size_t>(p) * kv_row + static_cast<size_t>(kh) * hd;
                            quant_kv_row(f.data() + o, hd, dst + o, sd[static_cast<size_t>(p) * nkv + kh]);
                        }
                    continue;
                }
                uint16_t *dst = L.kv.data() + static_cast<size_t>(kvi) * c.max_ctx * kv_row;
                for (size_t i = 0; i < f.size(); ++i) dst[i] = f32_to_f16(f[i]);
            }
        }
    }
    m->pos = ctx;
}

uint8_t *orc_model_tensor(orc_model *m, int kind, int layer, int expert, int64_t *bytes, float *globals) {
    auto ret = [&](auto &vec, float g0, float g1) -> uint8_t * {
        if (bytes) *bytes = static_cast<int64_t>(vec.size() * sizeof(vec[0]));
        if (globals) globals[0] = g0, globals[1] = g1;
        return reinterpret_cast<uint8_t *>(vec.data());
    };
    if (kind == ORC_EMBED) return ret(m->embed, m->g_embed, 0);
    if (kind == ORC_LM_HEAD) return ret(m->lm_head, m->g_lm, 0);
    if (kind == ORC_FINAL_NORM) return ret(m->final_norm, 0, 0);
    if (m->c.mtp) {
        if (kind == ORC_MTP_FC) return ret(m->mtp_fc, m->g_fc, 0);
        if (kind == ORC_MTP_NORM) return ret(m->mtp_norm, 0, 0);
        if (kind == ORC_MTP_PRE_E) return ret(m->mtp_pre_e, 0, 0);
        if (kind == ORC_MTP_PRE_H) return ret(m->mtp_pre_h, 0, 0);
    }
    if (layer < 0 || layer >= static_cast<int>(m->layers.size())) return nullptr;
    Layer &L = m->layers[static_cast<size_t>(layer)];
    switch (kind) {
    case ORC_IN_NORM: return ret(L.in_norm, 0, 0);
    case ORC_POST_NORM: return ret(L.post_norm, 0, 0);
    case ORC_Q: return ret(L.q, L.gq, 0);
    case ORC_K: return ret(L.k, L.gk, 0);
    case ORC_V: return ret(L.v, L.gv, 0);
    case ORC_O: return ret(L.o, L.go, 0);
    case ORC_Q_NORM: return ret(L.q_norm, 0, 0);
    case ORC_K_NORM: return ret(L.k_norm, 0, 0);
    case ORC_ROUTER: return ret(L.router, 0, 0);
    case ORC_SHARED_GATE: return ret(L.shared_gate, 0, 0);
    case ORC_SH_GATE: return ret(L.sh_gate, L.gsg, 0);
    case ORC_SH_UP: return ret(L.sh_up, L.gsu, 0);
    case ORC_SH_DOWN: return ret(L.sh_down, L.gsd, 0);
    case ORC_KV: return ret(L.kv, 0, 0);
    case ORC_KV8: return ret(L.kv8, 0, 0);
    case ORC_KVS: return ret(L.kvs, 0, 0);
    case ORC_GDN_QKV: return ret(L.gqkv, L.g_qkv, 0);
    case ORC_GDN_Z: return ret(L.gz, L.g_z, 0);
    case ORC_GDN_OUT: return ret(L.gout, L.g_out, 0);
    case ORC_GDN_A: return ret(L.ga, 0, 0);
    case ORC_GDN_B: return ret(L.gb, 0, 0);
    case ORC_GDN_ALOG: return ret(L.A_log, 0, 0);
    case ORC_GDN_DTB: return ret(L.dt_bias, 0, 0);
    case ORC_GDN_CONV: return ret(L.conv_w, 0, 0);
    case ORC_GDN_NORM: return ret(L.gnorm, 0, 0);
    case ORC_GDN_CONV_ST: return ret(L.conv_st, 0, 0);
    case ORC_GDN_S: return ret(L.S, 0, 0);
    case ORC_EXPERT: {
        if (expert < 0 || expert >= m->c.n_experts) return nullptr;
        const size_t eb = expert_block_bytes(m->c);
        if (bytes) *bytes = static_cast<int64_t>(eb);
        if (globals)
            globals[0] = L.expert_globals[static_cast<size_t>(2 * expert)],
            globals[1] = L.expert_globals[static_cast<size_t>(2 * expert + 1)];
        return L.experts.data() + eb * static_cast<size_t>(expert);
    }
    default: return nullptr;
    }
}

void orc_model_set_position(orc_model *m, int pos) { m->pos = pos; }
int orc_model_position(const orc_model *m) { return m->pos; }

const orc_config *orc_model_config(const orc_model *m) { return &m->c; }

int orc_model_verify(orc_model *m, const int32_t *tokens, int n, const int32_t *parents, int mode, float *logits,
                     int32_t *route_ids) {
    return orc_model_verify_trace(m, tokens, n, parents, mode, logits, route_ids, nullptr);
}

int orc_model_verify_trace(orc_model *m, const int32_t *tokens, int n, const int32_t *parents, int mode,
                           float *logits, int32_t *route_ids, float *trace) {
    const auto &c = m->c;
    const int H = c.hidden;
    if (n <= 0 || m->pos + n > c.max_ctx) return -1;
    for (int t = 0; t < n; ++t)
        if (tokens[t] < 0 || tokens[t] >= c.vocab) return -1;
    if (parents) {
        if (parents[0] != -1) return -1;
        for (int i = 1; i < n; ++i)
            if (parents[i] < 0 || parents[i] >= i) return -1;
    }
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<float> x(static_cast<size_t>(n) * H), h(static_cast<size_t>(n) * H), mix(static_cast<size_t>(n) * H);
    for (int t = 0; t < n; ++t)   // the embeddings: dequantized rows (pack.cpp:356-366)
        orc_dequant_rows(m->embed.data() + static_cast<size_t>(tokens[t]) * q4_row_bytes(H), 1, H, m->g_embed,
                         x.data() + static_cast<size_t>(t) * H);
    std::vector<int> ids(static_cast<size_t>(n) * c.top_k);
    for (int l = 0; l < c.n_layers; ++l) {
        Layer &L = m->layers[static_cast<size_t>(l)];
        float *tr = trace ? trace + static_cast<size_t>(l) * 4 * n * H : nullptr;   // [x in, x mid, h2, moe out]
        if (tr) std::copy(x.begin(), x.end(), tr);
        for (int t = 0; t < n; ++t)
            rmsnorm(x.data() + static_cast<size_t>(t) * H, L.in_norm.data(), h.data() + static_cast<size_t>(t) * H, H,
                    c.eps, true);
        if (L.gdn) gdn_layer(*m, L, n, h.data(), parents, mode, mix.data());
        else attention(*m, L, n, h.data(), m->pos, parents, mode, mix.data());
        for (int t = 0; t < n; ++t) {
            float *xr = x.data() + static_cast<size_t>(t) * H;
            const float *mr = mix.data() + static_cast<size_t>(t) * H;
            for (int i = 0; i < H; ++i) xr[i] += mr[i];
            rmsnorm(xr, L.post_norm.data(), h.data() + static_cast<size_t>(t) * H, H, c.eps, true);
        }
        if (tr) {
            std::copy(x.begin(), x.end(), tr + static_cast<size_t>(n) * H);
            std::copy(h.begin(), h.end(), tr + 2 * static_cast<size_t>(n) * H);
        }
        const orc_moe_weights w = moe_view(*m, L);
        moe_layer(w, n, h.data(), nullptr, mode, mix.data(), ids.data(), nullptr, nullptr);
        if (tr) std::copy(mix.begin(), mix.end(), tr + 3 * static_cast<size_t>(n) * H);
        if (route_ids)
            std::copy(ids.begin(), ids.end(), route_ids + static_cast<size_t>(l) * n * c.top_k);
        for (size_t i = 0; i < x.size(); ++i) x[i] += mix[i];
    }
    const auto t1 = std::chrono::steady_clock::now();
    for (int t = 0; t < n; ++t)
        rmsnorm(x.data() + static_cast<size_t>(t) * H, m->final_norm.data(), h.data() + static_cast<size_t>(t) * H, H,
                c.eps, true);
    const auto hs = crow_ptrs(h.data(), n, static_cast<size_t>(H));
    auto ls = row_ptrs(logits, n, static_cast<size_t>(c.vocab));
    matmul(m->lm_head.data(), c.vocab, H, m->g_lm, n, hs.data(), ls.data(), mode);
    m->hid = h;   // the final-normed rows: the MTP layer drafts from them (model.cpp:1580-1585)
    m->hid_rows.clear();
    const auto t2 = std::chrono::steady_clock::now();
    m->t_layers = std::chrono::duration<double>(t1 - t0).count();
    m->t_head = std::chrono::duration<double>(t2 - t1).count();
    m->last_pos = m->pos;
    m->last_n = n;
    m->pos += n;
    return 0;
}

int orc_model_keep(orc_model *m, int kept, const int32_t *path) {
    if (kept < 1 || kept > m->last_n || m->pos != m->last_pos + m->last_n) return -1;
    const auto &c = m->c;
    const size_t kv_row = static_cast<size_t>(c.n_kv_heads) * c.head_dim;
    if (path) {
        for (int j = 0; j < kept; ++j)
            if (path[j] < 0 || path[j] >= m->last_n || (j > 0 && path[j] <= path[j - 1])) return -1;
        const size_t nkv = static_cast<size_t>(c.n_kv_heads);
        for (int l = 0; l < c.n_layers; ++l) {   // (the MTP layer's KV is its own passes', not the verify's)
            Layer &L = m->layers[static_cast<size_t>(l)];
            for (int kvi = 0; kvi < 2; ++kvi)
                for (int j = 0; j < kept; ++j) {
                    if (path[j] == j) continue;
                    const size_t to = static_cast<size_t>(m->last_pos + j), from = static_cast<size_t>(m->last_pos + path[j]);
                    if (c.kv_int8) {
                        int8_t *base = L.kv8.data() + static_cast<size_t>(kvi) * c.max_ctx * kv_row;
                        float *sb = L.kvs.data() + static_cast<size_t>(kvi) * c.max_ctx * nkv;
                        std::memmove(base + to * kv_row, base + from * kv_row, kv_row);
                        std::memmove(sb + to * nkv, sb + from * nkv, nkv * sizeof(float));
                    } else {
                        uint16_t *base = L.kv.data() + static_cast<size_t>(kvi) * c.max_ctx * kv_row;
                        std::memmove(base + to * kv_row, base + from * kv_row, kv_row * 2);
                    }
                }
        }
    }
    // the Gated DeltaNet layers' states as after the last kept row (model.cpp:1617-1633)
    const int last = path ? path[kept - 1] : kept - 1;
    m->hid_rows.clear();
    if (path) m->hid_rows.assign(path, path + kept);
    for (auto &L : m->layers) {
        if (!L.gdn) continue;
        const size_t cs_n = L.conv_st.size(), s_n = L.S.size();
        std::copy(L.conv_bk.begin() + static_cast<ptrdiff_t>(last * cs_n), L.conv_bk.begin() + static_cast<ptrdiff_t>((last + 1) * cs_n),
                  L.conv_st.begin());
        std::copy(L.S_bk.begin() + static_cast<ptrdiff_t>(last * s_n), L.S_bk.begin() + static_cast<ptrdiff_t>((last + 1) * s_n),
                  L.S.begin());
    }
    m->pos = m->last_pos + kept;
    return 0;
}

int orc_model_hidden(const orc_model *m, float *out, int max_rows) {
    const int H = m->c.hidden, n = static_cast<int>(m->hid.size() / static_cast<size_t>(H));
    const int k = std::min(n, max_rows);
    std::copy(m->hid.begin(), m->hid.begin() + static_cast<ptrdiff_t>(k) * H, out);
    return k;
}

int orc_model_set_draft_vocab(orc_model *m, const int32_t *ids, int n) {
    const auto &c = m->c;
    if (n < 0 || (n > 0 && !ids)) return -1;
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= c.vocab) return -1;
    const size_t rb = q4_row_bytes(c.hidden);
    m->draft_ids.assign(ids, ids + n);
    m->draft_head.resize(static_cast<size_t>(n) * rb);
    for (int i = 0; i < n; ++i)   // model.cpp:812-818: the rows copied in the draft vocabulary's order
        std::memcpy(m->draft_head.data() + static_cast<size_t>(i) * rb, m->lm_head.data() + static_cast<size_t>(ids[i]) * rb, rb);
    return 0;
}

int orc_model_mtp(orc_model *m, const int32_t *toks, int n, int pos, const float *hidden, int mode, float *logits) {
    const auto &c = m->c;
    const int H = c.hidden;
    if (!c.mtp || n <= 0 || pos < 0 || pos + n > c.max_ctx) return -1;
    for (int t = 0; t < n; ++t)
        if (toks[t] < 0 || toks[t] >= c.vocab) return -1;
    std::vector<const float *> hs(static_cast<size_t>(n));
    for (int t = 0; t < n; ++t) {
        if (hidden) {
            hs[static_cast<size_t>(t)] = hidden + static_cast<size_t>(t) * H;
            continue;
        }
        const int r = m->hid_rows.empty() ? t : (t < static_cast<int>(m->hid_rows.size()) ? m->hid_rows[static_cast<size_t>(t)] : -1);
        if (r < 0 || static_cast<size_t>(r + 1) * H > m->hid.size()) return -1;
        hs[static_cast<size_t>(t)] = m->hid.data() + static_cast<size_t>(r) * H;
    }
    // the layer's input: [RMSNorm(embedding of the next token; 1 + pre_e) | RMSNorm(hidden; 1 + pre_h)], then fc
    std::vector<float> in(static_cast<size_t>(n) * 2 * H), e(static_cast<size_t>(H));
    for (int t = 0; t < n; ++t) {
        float *row = in.data() + static_cast<size_t>(t) * 2 * H;
        orc_dequant_rows(m->embed.data() + static_cast<size_t>(toks[t]) * q4_row_bytes(H), 1, H, m->g_embed, e.data());
        rmsnorm(e.data(), m->mtp_pre_e.data(), row, H, c.eps, true);
        rmsnorm(hs[static_cast<size_t>(t)], m->mtp_pre_h.data(), row + H, H, c.eps, true);
    }
    std::vector<float> x(static_cast<size_t>(n) * H), h(x.size()), mix(x.size());
    {
        const auto ins = crow_ptrs(in.data(), n, static_cast<size_t>(2 * H));
        auto xs = row_ptrs(x.data(), n, static_cast<size_t>(H));
        matmul(m->mtp_fc.data(), H, 2 * H, m->g_fc, n, ins.data(), xs.data(), mode);
    }
    // the decoder layer: attention over the MTP layer's own positions (slots pos..), then its MoE
    Layer &L = m->layers[static_cast<size_t>(c.n_layers)];
    for (int t = 0; t < n; ++t)
        rmsnorm(x.data() + static_cast<size_t>(t) * H, L.in_norm.data(), h.data() + static_cast<size_t>(t) * H, H, c.eps, true);
    attention(*m, L, n, h.data(), pos, nullptr, mode, mix.data());
    for (int t = 0; t < n; ++t) {
        float *xr = x.data() + static_cast<size_t>(t) * H;
        const float *mr = mix.data() + static_cast<size_t>(t) * H;
        for (int i = 0; i < H; ++i) xr[i] += mr[i];
        rmsnorm(xr, L.post_norm.data(), h.data() + static_cast<size_t>(t) * H, H, c.eps, true);
    }
    std::vector<int> ids(static_cast<size_t>(n) * c.top_k);
    const orc_moe_weights w = moe_view(*m, L);
    moe_layer(w, n, h.data(), nullptr, mode, mix.data(), ids.data(), nullptr, nullptr);
    for (size_t i = 0; i < x.size(); ++i) x[i] += mix[i];
    if (!logits) return 0;
    // the last row: mtp.norm, then lm_head (or the draft head)
    m->mtp_out.resize(static_cast<size_t>(H));
    rmsnorm(x.data() + static_cast<size_t>(n - 1) * H, m->mtp_norm.data(), m->mtp_out.data(), H, c.eps, true);
    const bool sub = !m->draft_ids.empty();
    const float *hp = m->mtp_out.data();
    matmul(sub ? m->draft_head.data() : m->lm_head.data(), sub ? static_cast<int64_t>(m->draft_ids.size()) : c.vocab, H,
           m->g_lm, 1, &hp, &logits, mode);
    return 0;
}

namespace {
// argmax (the first maximum, as std::max_element) and softmax_at (model.cpp:1286-1292): 1 / sum exp(double(l - max))
void pick_draft(const orc_model *m, const float *lg, int32_t *draft, float *prob) {
    const int rows = m->draft_ids.empty() ? m->c.vocab : static_cast<int>(m->draft_ids.size());
    int best = 0;
    for (int i = 1; i < rows; ++i)
        if (lg[i] > lg[best]) best = i;
    double sum = 0.0;
    for (int i = 0; i < rows; ++i) sum += std::exp(static_cast<double>(lg[i] - lg[best]));
    if (draft) *draft = m->draft_ids.empty() ? best : m->draft_ids[static_cast<size_t>(best)];
    if (prob) *prob = static_cast<float>(1.0 / sum);
}
}  // namespace

int orc_model_draft(orc_model *m, const int32_t *toks, int n, int pos, const float *hidden, int mode, float *logits,
                    int32_t *draft, float *prob) {
    std::vector<float> lg(static_cast<size_t>(m->c.vocab));
    if (orc_model_mtp(m, toks, n, pos, hidden, mode, lg.data()) != 0) return -1;
    pick_draft(m, lg.data(), draft, prob);
    const int rows = m->draft_ids.empty() ? m->c.vocab : static_cast<int>(m->draft_ids.size());
    if (logits) std::copy(lg.begin(), lg.begin() + rows, logits);
    return 0;
}

int orc_model_draft_next(orc_model *m, int32_t tok, int pos, int mode, float *logits, int32_t *draft, float *prob) {
    if (m->mtp_out.empty()) return -1;   // no MTP pass to go on from
    const std::vector<float> h = m->mtp_out;
    return orc_model_draft(m, &tok, 1, pos, h.data(), mode, logits, draft, prob);
}

void orc_model_last_times(const orc_model *m, double *t_layers, double *t_head) {
    if (t_layers) *t_layers = m->t_layers;
    if (t_head) *t_head = m->t_head;
}

}  // extern "C"
