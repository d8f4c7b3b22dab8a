// oracle_sample.cpp - the sampler and the two acceptance rules on the CPU.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP path, never part of it.
//
// Pinning (tests/test_oracle_sample.py): orc_sample_seeded against the reference's Sampler built from its sources
// (oracle/_ref: the same mt19937_64 stream, bit for bit); orc_sample with injected uniforms against the same
// candidates/top-p arithmetic in float64 numpy and the top-p prefix property; orc_accept_match by a brute-force
// loop; orc_accept_textbook by exhaustive enumeration on a tiny vocabulary (the output distribution equals p
// exactly, Leviathan et al. 2023 Thm 1) and a chi-square test over seeded uniforms.
#include <algorithm>
#include <cmath>
#include <random>
#include <utility>
#include <vector>

#include "oracle.h"
#include "oracle_internal.hpp"

namespace orc {
namespace {

struct Nucleus {
    std::vector<std::pair<float, int>> cand;   // (e, index) in descending logit order
    size_t keep = 0;
    double sum = 0.0, kept = 0.0;
};

// sampler.cpp:18-41: candidates (top_k, else the cap; cap 0 = every token) sorted by logit descending (ties to the
// lower index: the reference's partial_sort leaves them unspecified), e = exp((l - max) / T) in float, their sum in
// double, top-p the smallest prefix whose probability reaches p
Nucleus nucleus(const float *logits, int n, float temperature, float top_p, int top_k, int cap) {
    Nucleus nu;
    const int k = std::min(n, top_k > 0 ? top_k : (cap > 0 ? cap : n));
    nu.cand.resize(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) nu.cand[static_cast<size_t>(i)] = {logits[i], i};
    std::partial_sort(nu.cand.begin(), nu.cand.begin() + k, nu.cand.end(), [](const auto &a, const auto &b) {
        return a.first > b.first || (a.first == b.first && a.second < b.second);
    });
    nu.cand.resize(static_cast<size_t>(k));
    const float mx = nu.cand[0].first;
    for (auto &c : nu.cand) {
        c.first = std::exp((c.first - mx) / temperature);
        nu.sum += c.first;
    }
    nu.keep = nu.cand.size();
    if (top_p < 1.0f) {
        double acc = 0.0;
        for (size_t i = 0; i < nu.cand.size(); ++i) {
            acc += nu.cand[i].first / nu.sum;
            if (acc >= top_p) {
                nu.keep = i + 1;
                break;
            }
        }
    }
    for (size_t i = 0; i < nu.keep; ++i) nu.kept += nu.cand[i].first;
    return nu;
}

// sampler.cpp:44-49 with r = kept * u (uniform_real_distribution<double>(0, kept) of a canonical u)
int draw(const Nucleus &nu, double u) {
    double r = nu.kept * u;
    for (size_t i = 0; i < nu.keep; ++i) {
        r -= nu.cand[i].first;
        if (r <= 0.0) return nu.cand[i].second;
    }
    return nu.cand[nu.keep - 1].second;
}

int argmax(const float *logits, int n) { return static_cast<int>(std::max_element(logits, logits + n) - logits); }

int sample(const float *logits, int n, float temperature, float top_p, int top_k, int cap, double u) {
    if (temperature <= 0.0f) return argmax(logits, n);   // sampler.cpp:17
    return draw(nucleus(logits, n, temperature, top_p, top_k, cap), u);
}

// probability of token x under the nucleus (0 outside it)
double prob(const Nucleus &nu, int x) {
    for (size_t i = 0; i < nu.keep; ++i)
        if (nu.cand[i].second == x) return nu.cand[i].first / nu.kept;
    return 0.0;
}

}  // namespace
}  // namespace orc

using namespace orc;

extern "C" {

int orc_sample(const float *logits, int n, float temperature, float top_p, int top_k, int cap, double u) {
    return sample(logits, n, temperature, top_p, top_k, cap, u);
}

void orc_sample_seeded(const float *logits, int n, float temperature, float top_p, int top_k, uint64_t seed,
                       int draws, int32_t *out) {
    std::mt19937_64 rng(seed);
    for (int d = 0; d < draws; ++d) {
        if (temperature <= 0.0f) {
            out[d] = argmax(logits, n);
            continue;
        }
        const Nucleus nu = nucleus(logits, n, temperature, top_p, top_k, 1024);
        double r = std::uniform_real_distribution<double>(0.0, nu.kept)(rng);
        int pick = nu.cand[nu.keep - 1].second;
        for (size_t i = 0; i < nu.keep; ++i) {
            r -= nu.cand[i].first;
            if (r <= 0.0) {
                pick = nu.cand[i].second;
                break;
            }
        }
        out[d] = pick;
    }
}

// geode.cpp:236-255 and :331-350 as written: `seen` holds the answer's distinct tokens so far (in order), each row's
// logits lose presence_penalty at every seen token before it is sampled, a sampled token joins `seen` once, and a draft
// stands while the row before samples exactly it and it is no stop token. logits are modified in place (as there).
int orc_accept_match_ex(float *logits, int V, const int32_t *batch, int n, float temperature, float top_p, int top_k,
                        int cap, const double *u, const int32_t *seen_in, int n_seen, float presence_penalty,
                        const int32_t *stop, int n_stop, int32_t *out, int *kept) {
    std::vector<int32_t> seen;
    std::vector<uint8_t> is_seen(presence_penalty != 0.0f ? static_cast<size_t>(V) : 0, 0);
    if (!is_seen.empty())
        for (int j = 0; j < n_seen; ++j) {
            const int32_t t = seen_in[j];
            if (t >= 0 && t < V && !is_seen[static_cast<size_t>(t)]) {
                is_seen[static_cast<size_t>(t)] = 1;
                seen.push_back(t);
            }
        }
    auto is_stop = [&](int32_t t) {
        for (int j = 0; j < n_stop; ++j)
            if (stop[j] == t) return true;
        return false;
    };
    int emitted = 0, k = 1;
    for (int i = 0; i < n; ++i) {
        float *lg = logits + static_cast<size_t>(i) * V;
        for (int32_t t : seen) lg[static_cast<size_t>(t)] -= presence_penalty;
        const int y = sample(lg, V, temperature, top_p, top_k, cap, u[i]);
        if (!is_seen.empty() && y >= 0 && y < V && !is_seen[static_cast<size_t>(y)]) {
            is_seen[static_cast<size_t>(y)] = 1;
            seen.push_back(y);
        }
        out[emitted++] = y;
        if (i + 1 < n && y == batch[i + 1] && !is_stop(y)) {   // the draft stands (geode.cpp:333)
            ++k;
            continue;
        }
        break;
    }
    if (kept) *kept = k;
    return emitted;
}

int orc_accept_match(const float *logits, int V, const int32_t *batch, int n, float temperature, float top_p,
                     int top_k, int cap, const double *u, int32_t *out, int *kept) {
    int emitted = 0, k = 1;
    for (int i = 0; i < n; ++i) {
        const int y = sample(logits + static_cast<size_t>(i) * V, V, temperature, top_p, top_k, cap, u[i]);
        out[emitted++] = y;
        if (i + 1 < n && y == batch[i + 1]) {   // the draft stands (geode.cpp:333)
            ++k;
            continue;
        }
        break;
    }
    if (kept) *kept = k;
    return emitted;
}

void orc_nucleus_probs(const float *logits, int V, float temperature, float top_p, double *probs) {
    const Nucleus nu = nucleus(logits, V, temperature, top_p, 0, 0);
    std::fill(probs, probs + V, 0.0);
    for (size_t i = 0; i < nu.keep; ++i) probs[nu.cand[i].second] = nu.cand[i].first / nu.kept;
}

int orc_accept_textbook(const float *target, const float *draft, int V, int k, float temperature, float top_p,
                        int greedy, const float *u_draft, const float *u_acc, float u_res, int32_t *out) {
    int emitted = 0;
    for (int i = 0; i < k; ++i) {
        const float *tl = target + static_cast<size_t>(i) * V, *dl = draft + static_cast<size_t>(i) * V;
        if (greedy) {
            const int d = argmax(dl, V), y = argmax(tl, V);
            out[emitted++] = y;
            if (y != d) return emitted;
            continue;
        }
        const Nucleus p = nucleus(tl, V, temperature, top_p, 0, 0), q = nucleus(dl, V, temperature, top_p, 0, 0);
        const int d = draw(q, static_cast<double>(u_draft[i]));
        const double pd = prob(p, d), qd = prob(q, d);
        if (static_cast<double>(u_acc[i]) * qd < pd) {   // accepted with probability min(1, p/q)
            out[emitted++] = d;
            continue;
        }
        // rejected: a token from max(0, p - q), normalised, by inverse CDF in index order
        std::vector<double> pp(static_cast<size_t>(V), 0.0), qq(static_cast<size_t>(V), 0.0);
        for (size_t j = 0; j < p.keep; ++j) pp[static_cast<size_t>(p.cand[j].second)] = p.cand[j].first / p.kept;
        for (size_t j = 0; j < q.keep; ++j) qq[static_cast<size_t>(q.cand[j].second)] = q.cand[j].first / q.kept;
        double total = 0.0;
        for (int x = 0; x < V; ++x) total += std::max(0.0, pp[static_cast<size_t>(x)] - qq[static_cast<size_t>(x)]);
        if (!(total > 0.0)) {
            out[emitted++] = draw(p, static_cast<double>(u_res));
            return emitted;
        }
        const double goal = static_cast<double>(u_res) * total;
        double acc = 0.0;
        int pick = -1, last = -1;
        for (int x = 0; x < V; ++x) {
            const double r = std::max(0.0, pp[static_cast<size_t>(x)] - qq[static_cast<size_t>(x)]);
            if (r <= 0.0) continue;
            last = x;
            acc += r;
            if (acc >= goal) {
                pick = x;
                break;
            }
        }
        out[emitted++] = pick >= 0 ? pick : last;
        return emitted;
    }
    // every draft stood: the bonus token from the last target row
    const float *tl = target + static_cast<size_t>(k) * V;
    if (greedy) {
        out[emitted++] = argmax(tl, V);
    } else {
        out[emitted++] = draw(nucleus(tl, V, temperature, top_p, 0, 0), static_cast<double>(u_res));
    }
    return emitted;
}

}  // extern "C"
