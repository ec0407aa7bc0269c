// The host half of beam search (src/translator.rs:250-335): per step, merge the top-k
// (log-prob, token) of every decoder row into the next alive hypotheses, the finished
// ones and the row reorder + next input of the following step.  The device side (the
// decoder step and the log-softmax + top-k) lives in runtime.cpp; this part is plain
// host code, shared by Model::beam and mlg_beam_search_host.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace mlg {

class BeamMerge {
  public:
    // b sentences of k beams each (decoder row s * k + i is beam i of sentence s).
    BeamMerge(int b, int k, int max_new, float length_penalty, uint32_t eos);
    // Step `step` (1-based) from vals/idx [b * k][k]: the top-k log-probs and tokens of
    // every row, best first.  Returns true when decoding ends after this step
    // (step == max_new, or every sentence is done, translator.rs:320-322); otherwise
    // reorder()/next() hold the next step's rows: row r continues row reorder()[r] and is
    // fed next()[r].
    bool merge(int step, const float *vals, const uint32_t *idx);
    const std::vector<uint32_t> &reorder() const { return reorder_; }
    const std::vector<uint32_t> &next() const { return next_; }
    // Best finished hypothesis per sentence (the alive ones if none finished), by
    // Iterator::max_by under total_cmp: the last of equal maxima (translator.rs:327-334).
    std::vector<std::vector<uint32_t>> result() const;

  private:
    struct Hyp {
        float score;
        std::vector<uint32_t> toks;
    };
    float penalty(size_t len) const;
    int b_, k_, max_new_;
    float lp_;
    uint32_t eos_;
    std::vector<std::vector<Hyp>> alive_, done_;
    std::vector<uint8_t> is_done_;
    std::vector<uint32_t> reorder_, next_;
};

}  // namespace mlg
