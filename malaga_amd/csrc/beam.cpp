// src/translator.rs:250-335, the host merge of beam search.
#include "beam.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace mlg {

namespace {
// f32::total_cmp's order (IEEE 754 totalOrder): -NaN < -inf < ... < -0 < +0 < ... < +inf < NaN.
// Flipping the magnitude bits of negative values makes the signed integer order that order.
int32_t total_key(float f) {
    int32_t i;
    std::memcpy(&i, &f, 4);
    return i ^ int32_t(uint32_t(i >> 31) >> 1);
}
}  // namespace

BeamMerge::BeamMerge(int b, int k, int max_new, float length_penalty, uint32_t eos)
    : b_(b), k_(k), max_new_(max_new), lp_(length_penalty), eos_(eos), alive_(size_t(b)), done_(size_t(b)),
      is_done_(size_t(b), 0) {
    // only beam 0 starts alive (translator.rs:264-265)
    for (auto &a : alive_) a.push_back(Hyp{0.f, {}});
}

// translator.rs:269: len.max(1) ^ length_penalty
float BeamMerge::penalty(size_t len) const { return std::pow(float(std::max<size_t>(len, 1)), lp_); }

bool BeamMerge::merge(int step, const float *vals, const uint32_t *idx) {
    reorder_.clear();
    next_.clear();
    struct Cand {
        float score;
        int bi;
        uint32_t tok;
    };
    std::vector<Cand> cands;
    for (int sn = 0; sn < b_; ++sn) {
        // every alive beam's k continuations, best first by total_cmp; the stable sort
        // keeps equal scores in beam-then-rank order (translator.rs:277-284)
        cands.clear();
        for (int bi = 0; bi < int(alive_[sn].size()); ++bi) {
            const size_t row = size_t(sn) * k_ + bi;
            for (int j = 0; j < k_; ++j)
                cands.push_back({alive_[sn][bi].score + vals[row * k_ + j], bi, idx[row * k_ + j]});
        }
        std::stable_sort(cands.begin(), cands.end(),
                         [](const Cand &a, const Cand &c) { return total_key(a.score) > total_key(c.score); });
        std::vector<Hyp> next_alive;
        for (const Cand &cd : cands) {
            if (int(next_alive.size()) == k_) break;
            std::vector<uint32_t> toks = alive_[sn][cd.bi].toks;
            // EOS, or any token at the last step, finishes the hypothesis (translator.rs:291-299);
            // its length counts the EOS (tokens + 1)
            if (cd.tok == eos_ || step == max_new_) {
                if (cd.tok != eos_) toks.push_back(cd.tok);
                const size_t len = toks.size() + 1;
                if (!is_done_[sn]) done_[sn].push_back({cd.score / penalty(len), std::move(toks)});
                continue;
            }
            toks.push_back(cd.tok);
            reorder_.push_back(uint32_t(sn * k_ + cd.bi));
            next_.push_back(cd.tok);
            next_alive.push_back({cd.score, std::move(toks)});
        }
        // translator.rs:306-311: stop once k hypotheses are done and the best of them is
        // at least the best alive one normalized as if it ended at the next step
        float best_done = -INFINITY;
        for (const Hyp &h : done_[sn]) best_done = std::max(best_done, h.score);
        const float best_alive = next_alive.empty() ? -INFINITY : next_alive[0].score / penalty(size_t(step) + 1);
        if (int(done_[sn].size()) >= k_ && best_done >= best_alive) is_done_[sn] = 1;
        // translator.rs:312-317: rectangular batch, copies of beam 0 fed EOS, scored -inf
        while (int(next_alive.size()) < k_) {
            reorder_.push_back(uint32_t(sn * k_));
            next_.push_back(eos_);
            next_alive.push_back({-INFINITY, {}});
        }
        alive_[sn] = std::move(next_alive);
    }
    return step == max_new_ || std::all_of(is_done_.begin(), is_done_.end(), [](uint8_t v) { return v != 0; });
}

std::vector<std::vector<uint32_t>> BeamMerge::result() const {
    std::vector<std::vector<uint32_t>> res(static_cast<size_t>(b_));
    for (int sn = 0; sn < b_; ++sn) {
        const auto &list = done_[sn].empty() ? alive_[sn] : done_[sn];
        int best = -1;
        for (int i = 0; i < int(list.size()); ++i)
            if (best < 0 || total_key(list[i].score) >= total_key(list[best].score)) best = i;
        if (best >= 0) res[sn] = list[best].toks;
    }
    return res;
}

}  // namespace mlg
