// Host-side token selection of the worker path: the reference's sampler
// (engine/src/sampling.cpp) over the logits or the candidate result one
// decode step returns.  A request carries a seed, and the same seed must draw
// the same token from the same logits, so each function keeps the reference's
// float operations in their order (this file is built without contraction),
// its standard-library selection and sort, and std::mt19937 with
// uniform_real_distribution<float> as the generator.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <random>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "engine_err.h"
#include "vgx.h"
#include "vgx_engine.h"

struct vgx_sampler {
    std::mt19937 rng;
};

namespace {

using Prob = std::pair<float, int>;  // (probability, token)

bool by_prob(const Prob& a, const Prob& b) { return a.first > b.first; }

// The distribution a draw uses (keep_distribution, engine/src/sampling.cpp:
// 66-117): softmax at temperature T, a top_k cut renormalised to mass 1,
// then the shortest prefix of the descending list whose mass reaches top_p
// (its mass is `mass`).  T <= 0 is the first maximum with probability 1.
std::vector<Prob> kept(const float* logits, int n, float temp, float top_p, int top_k, float* mass) {
    std::vector<Prob> p;
    if (temp <= 0.0f) {
        int best = 0;
        for (int i = 1; i < n; ++i)
            if (logits[i] > logits[best]) best = i;
        p.emplace_back(1.0f, best);
        *mass = 1.0f;
        return p;
    }
    p.resize((size_t)n);
    float mx = -1e30f;
    for (int i = 0; i < n; ++i) mx = std::max(mx, logits[i] / temp);
    float total = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float e = expf(logits[i] / temp - mx);
        p[(size_t)i] = Prob(e, i);
        total += e;
    }
    for (Prob& x : p) x.first /= total;
    if (top_k > 0 && top_k < n) {
        std::nth_element(p.begin(), p.begin() + top_k, p.end(), by_prob);
        std::sort(p.begin(), p.begin() + top_k, by_prob);
        p.resize((size_t)top_k);
        float m = 0.0f;
        for (const Prob& x : p) m += x.first;
        if (m > 0.0f)
            for (Prob& x : p) x.first /= m;
    } else {
        std::sort(p.begin(), p.end(), by_prob);
    }
    float c = 0.0f;
    size_t cut = 0;
    while (cut < p.size()) {
        c += p[cut].first;
        ++cut;
        if (c >= top_p) break;
    }
    p.resize(cut);
    *mass = c;
    return p;
}

float uniform01(std::mt19937& rng) { return std::uniform_real_distribution<float>(0.0f, 1.0f)(rng); }

}  // namespace

extern "C" {

int vgx_sampler_create(uint32_t seed, vgx_sampler** out) {
    engine_clear_error();
    if (!out) return engine_fail(VGX_EINVAL, "vgx_sampler_create: NULL argument");
    *out = new vgx_sampler{std::mt19937(seed)};
    return VGX_OK;
}

int vgx_sampler_free(vgx_sampler* s) {
    delete s;
    return VGX_OK;
}

int vgx_sample_logits(vgx_sampler* s, const float* logits, int n, float temp, float top_p, int top_k, int* token,
                      float* logprob) {
    engine_clear_error();
    if (!s || !logits || !token) return engine_fail(VGX_EINVAL, "vgx_sample_logits: NULL argument");
    if (n <= 0) return engine_fail(VGX_EINVAL, "vgx_sample_logits: empty logits");
    float mass = 0.0f;
    const std::vector<Prob> d = kept(logits, n, temp, top_p, top_k, &mass);
    const float r = uniform01(s->rng) * mass;
    // the first kept token whose running mass reaches r; the last if rounding
    // leaves r above them all (sample_token / sample_token_report,
    // engine/src/sampling.cpp:119-142)
    Prob pick = d.back();
    float acc = 0.0f;
    for (const Prob& x : d) {
        acc += x.first;
        if (r <= acc) {
            pick = x;
            break;
        }
    }
    *token = pick.second;
    if (logprob) *logprob = logf(mass > 0.0f ? pick.first / mass : pick.first);
    return VGX_OK;
}

int vgx_argmax_report(const float* logits, int n, int* token, float* logprob) {
    engine_clear_error();
    if (!logits || !token) return engine_fail(VGX_EINVAL, "vgx_argmax_report: NULL argument");
    if (n <= 0) return engine_fail(VGX_EINVAL, "vgx_argmax_report: empty logits");
    // argmax_token_report (engine/src/sampling.cpp:144-155): the first
    // maximum and its log-probability under the untempered softmax
    int best = 0;
    float mx = logits[0];
    for (int i = 1; i < n; ++i) {
        if (logits[i] > logits[best]) best = i;
        mx = std::max(mx, logits[i]);
    }
    double total = 0.0;
    for (int i = 0; i < n; ++i) total += exp((double)logits[i] - mx);
    *token = best;
    if (logprob) *logprob = (float)(((double)logits[best] - mx) - log(total));
    return VGX_OK;
}

int vgx_sample_candidates(vgx_sampler* s, const float* value, const int* cand_token, int n, int strict,
                          float logsumexp, float temp, float top_p, int top_k, int* token) {
    engine_clear_error();
    if (!s || !token || (n > 0 && (!value || !cand_token)))
        return engine_fail(VGX_EINVAL, "vgx_sample_candidates: NULL argument");
    // sample_candidate_result (engine/src/sampling.cpp:164-199)
    if (n <= 0) {
        *token = 2;
        return VGX_OK;
    }
    if (temp <= 0.0f) {
        int best = 0;
        for (int i = 1; i < n; ++i)
            if (value[i] > value[best]) best = i;
        *token = cand_token[best];
        return VGX_OK;
    }
    std::vector<Prob> c((size_t)n);
    if (strict) {
        for (int i = 0; i < n; ++i) c[(size_t)i] = Prob(expf(value[i] / temp - logsumexp), cand_token[i]);
    } else {
        float mx = -1e30f;
        for (int i = 0; i < n; ++i) mx = std::max(mx, value[i] / temp);
        float total = 0.0f;
        for (int i = 0; i < n; ++i) {
            c[(size_t)i] = Prob(expf(value[i] / temp - mx), cand_token[i]);
            total += c[(size_t)i].first;
        }
        for (Prob& x : c) x.first /= total;
    }
    std::sort(c.begin(), c.end(), by_prob);
    const int kmax = (top_k > 0 && top_k < n) ? top_k : n;
    if (top_k > 0) {
        float m = 0.0f;
        for (int i = 0; i < kmax; ++i) m += c[(size_t)i].first;
        if (m > 0.0f)
            for (int i = 0; i < kmax; ++i) c[(size_t)i].first /= m;
    }
    float cdf = 0.0f;
    int cut = 0;
    while (cut < kmax) {
        cdf += c[(size_t)cut].first;
        ++cut;
        if (cdf >= top_p) break;
    }
    const float x = uniform01(s->rng) * cdf;
    float acc = 0.0f;
    for (int i = 0; i < cut; ++i) {
        acc += c[(size_t)i].first;
        if (x <= acc) {
            *token = c[(size_t)i].second;
            return VGX_OK;
        }
    }
    *token = c[(size_t)cut - 1].second;
    return VGX_OK;
}

int vgx_apply_penalties(float* logits, int n, const int* recent, int nrecent, float repetition, float frequency,
                        float presence, int no_repeat_ngram, float min_p) {
    engine_clear_error();
    if (!logits || (nrecent > 0 && !recent)) return engine_fail(VGX_EINVAL, "vgx_apply_penalties: NULL argument");
    // apply_sampling_penalties (engine/src/sampling.cpp:16-56), with the
    // process-wide settings passed in
    if (nrecent <= 0 && min_p <= 0.0f) return VGX_OK;
    std::unordered_map<int, int> counts;
    for (int i = 0; i < nrecent; ++i) ++counts[recent[i]];
    if (repetition != 1.0f) {
        for (const auto& kv : counts) {
            const int t = kv.first;
            if (t < 0 || t >= n) continue;
            if (logits[t] > 0) logits[t] /= repetition;
            else logits[t] *= repetition;
        }
    }
    if (frequency != 0.0f || presence != 0.0f) {
        for (const auto& kv : counts) {
            const int t = kv.first;
            if (t < 0 || t >= n) continue;
            logits[t] -= frequency * kv.second;
            logits[t] -= presence;
        }
    }
    // an n-gram that would repeat: the token that followed each earlier
    // occurrence of the last n-1 tokens is banned
    const int g = no_repeat_ngram;
    if (g > 1 && nrecent >= g) {
        const int* tail = recent + nrecent - (g - 1);
        for (int i = 0; i + g < nrecent; ++i) {
            bool match = true;
            for (int j = 0; j < g - 1 && match; ++j) match = recent[i + j] == tail[j];
            if (match) {
                const int banned = recent[i + g - 1];
                if (banned >= 0 && banned < n) logits[banned] = -1e30f;
            }
        }
    }
    if (min_p > 0.0f) {
        float mx = -1e30f;
        for (int i = 0; i < n; ++i) mx = std::max(mx, logits[i]);
        const float cutoff = mx + logf(min_p);
        for (int i = 0; i < n; ++i)
            if (logits[i] < cutoff) logits[i] = -1e30f;
    }
    return VGX_OK;
}

}  // extern "C"
