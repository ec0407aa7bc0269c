#include "server.hpp"

#include <algorithm>
#include <chrono>
#include <tuple>

namespace mlg {

namespace {
[[noreturn]] void fail_invalid(const char *msg) { throw Failure{ERR_INVALID, msg}; }
}  // namespace

void Job::finish(int st, std::string err, std::vector<std::vector<uint32_t>> rows) {
    {
        std::lock_guard<std::mutex> lk(mu);
        status = st;
        error = std::move(err);
        out = std::move(rows);
        done = true;
    }
    cv.notify_all();
}

bool Job::wait(int timeout_ms) {
    std::unique_lock<std::mutex> lk(mu);
    if (timeout_ms < 0) {
        cv.wait(lk, [&] { return done; });
        return true;
    }
    return cv.wait_for(lk, std::chrono::milliseconds(timeout_ms), [&] { return done; });
}

Server::Server(Model &m, const GenOptions &defaults) : m_(m), defaults_(defaults) {
    thread_ = std::thread([this] { loop(); });
}

Server::~Server() {
    {
        std::lock_guard<std::mutex> lk(mu_);
        stop_ = true;
    }
    cv_.notify_all();
    if (thread_.joinable()) thread_.join();
}

std::shared_ptr<Job> Server::submit(std::vector<std::vector<uint32_t>> src, uint32_t src_lang, uint32_t tgt_lang,
                                    int beam, const std::string &shortlist) {
    const ModelConfig &c = m_.cfg;
    if (tgt_lang >= uint32_t(c.vocab_size)) fail_invalid("target language id out of range");
    for (const auto &r : src) {
        if (r.empty()) fail_invalid("empty source row");
        if (int(r.size()) > c.max_position_embeddings) fail_invalid("source longer than the position table");
        for (uint32_t t : r)
            if (t >= uint32_t(c.vocab_size)) fail_invalid("token id out of range");
    }
    auto j = std::make_shared<Job>();
    j->src = std::move(src);
    j->src_lang = src_lang;
    j->tgt_lang = tgt_lang;
    j->beam = std::clamp(beam > 0 ? beam : defaults_.beam_size, 1, 8);
    j->shortlist = shortlist;
    if (j->src.empty()) {  // nothing to decode: answered at once
        j->finish(OK, "", {});
        std::lock_guard<std::mutex> lk(mu_);
        ++stats_.jobs;
        return j;
    }
    {
        std::lock_guard<std::mutex> lk(mu_);
        if (stop_) fail_invalid("server stopped");
        queue_.push_back(j);
    }
    cv_.notify_one();
    return j;
}

ServerStats Server::stats() const {
    std::lock_guard<std::mutex> lk(mu_);
    return stats_;
}

void Server::loop() {
    (void)hipSetDevice(m_.ctx->device);  // the current device is per thread
    for (;;) {
        std::vector<std::shared_ptr<Job>> jobs;
        {
            std::unique_lock<std::mutex> lk(mu_);
            cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
            if (queue_.empty()) return;  // stopped and drained
            jobs.assign(queue_.begin(), queue_.end());
            queue_.clear();
        }
        // server.rs:83-90: the group of the oldest job's key, then the rest, in order
        while (!jobs.empty()) {
            auto key = [](const Job &j) { return std::tie(j.src_lang, j.tgt_lang, j.beam, j.shortlist); };
            std::vector<std::shared_ptr<Job>> group, rest;
            for (auto &j : jobs) (key(*j) == key(*jobs[0]) ? group : rest).push_back(j);
            run_group(group);
            jobs = std::move(rest);
        }
    }
}

// server.rs:93-112: every sentence of every job of the group in one translate_batch
// call; each job receives its own rows, or the group's error.
void Server::run_group(const std::vector<std::shared_ptr<Job>> &group) {
    std::vector<std::vector<uint32_t>> src;
    for (const auto &j : group) src.insert(src.end(), j->src.begin(), j->src.end());
    GenOptions o = defaults_;
    o.beam_size = group[0]->beam;
    o.shortlist = group[0]->shortlist;
    int st = OK;
    std::string err;
    std::vector<std::vector<uint32_t>> out;
    try {
        std::lock_guard<std::mutex> lk(m_.ctx->mu);
        out = generate(m_, src, group[0]->tgt_lang, o);
    } catch (const Failure &f) {
        st = f.code;
        err = f.msg;
    } catch (const std::bad_alloc &) {
        st = ERR_OOM;
        err = "OUT_OF_MEMORY: host allocation failed";
    } catch (const std::exception &e) {
        st = ERR_INVALID;
        err = e.what();
    }
    {
        std::lock_guard<std::mutex> lk(mu_);
        stats_.jobs += int64_t(group.size());
        stats_.groups += 1;
        stats_.sentences += int64_t(src.size());
        stats_.largest_group = std::max<int64_t>(stats_.largest_group, int64_t(src.size()));
    }
    size_t k = 0;
    for (const auto &j : group) {
        if (st != OK) {
            j->finish(st, err, {});
            continue;
        }
        std::vector<std::vector<uint32_t>> rows(out.begin() + k, out.begin() + k + j->src.size());
        k += j->src.size();
        j->finish(OK, "", std::move(rows));
    }
}

}  // namespace mlg
