// Dynamic batching front end of the decode path (crates/malaga/src/server.rs:74-112):
// one inference thread owns the model; callers on any thread enqueue jobs; the thread
// takes every job already queued, groups those with the same (source language,
// target language, beam size, shortlist) in order of first arrival, and decodes each
// group as one translate_batch call, so requests that arrive while the GPU is busy
// share the next batch.
#pragma once
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "runtime.hpp"

namespace mlg {

struct Job {
    std::vector<std::vector<uint32_t>> src;
    uint32_t src_lang = 0, tgt_lang = 0;
    int beam = 1;
    std::string shortlist;
    // result, set once by the inference thread
    std::mutex mu;
    std::condition_variable cv;
    bool done = false;
    int status = OK;
    std::string error;
    std::vector<std::vector<uint32_t>> out;

    void finish(int st, std::string err, std::vector<std::vector<uint32_t>> rows);
    // Waits up to timeout_ms (< 0: without limit); true once the job is done.
    bool wait(int timeout_ms);
};

struct ServerStats {
    int64_t jobs = 0, groups = 0, sentences = 0, largest_group = 0;  // largest_group in sentences
};

class Server {
  public:
    // defaults: options of every group except beam_size and shortlist, which come
    // with each job (server.rs:86-88).  The model must outlive the server.
    Server(Model &m, const GenOptions &defaults);
    ~Server();  // finishes every queued job, then joins the inference thread
    // Validates and enqueues one job (beam <= 0: the defaults' beam size; clamped to
    // 1..8 as server.rs:64 does).  Throws Failure(ERR_INVALID) on bad input.
    std::shared_ptr<Job> submit(std::vector<std::vector<uint32_t>> src, uint32_t src_lang, uint32_t tgt_lang,
                                int beam, const std::string &shortlist);
    ServerStats stats() const;

  private:
    void loop();
    void run_group(const std::vector<std::shared_ptr<Job>> &group);
    Model &m_;
    GenOptions defaults_;
    mutable std::mutex mu_;
    std::condition_variable cv_;
    std::deque<std::shared_ptr<Job>> queue_;
    bool stop_ = false;
    ServerStats stats_;
    std::thread thread_;
};

}  // namespace mlg
