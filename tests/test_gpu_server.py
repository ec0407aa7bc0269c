"""Dynamic batching caller (crates/malaga/src/server.rs:74-112) on the GPU: jobs from
several threads are grouped by (source, target, beam, shortlist) and decoded together;
each job's rows equal the oracle's translation of that job alone (batching
independence, as pipeline.rs:44-57 asserts for F32)."""
import threading

import numpy as np
import pytest

import malaga_amd as M
from malaga_amd import MalagaError
import oracle as O
from tests.conftest import pipeline_sentences

pytestmark = pytest.mark.gpu
PLT, OTHER = 256, 255  # two target-language tokens of the tiny vocabulary


@pytest.fixture(scope="module")
def tiny(tiny_gguf):
    p = tiny_gguf("f32")
    T = M.Translator.load(p)
    yield T, O.Model(p)
    T.close()


def _jobs(seed, n_jobs):
    rng = np.random.default_rng(seed)
    base = pipeline_sentences()
    jobs = []
    for i in range(n_jobs):
        k = int(rng.integers(1, 4))
        src = [base[int(j)] for j in rng.integers(0, len(base), k)]
        jobs.append((src, PLT if i % 3 else OTHER))
    return jobs


def test_concurrent_submitters_match_oracle(tiny):
    T, orc = tiny
    srv = M.Server(T)
    jobs = _jobs(1, 24)
    results = [None] * len(jobs)

    def client(idx):
        for i in idx:
            src, tgt = jobs[i]
            results[i] = srv.submit(src, tgt, src_lang=254).result()

    threads = [threading.Thread(target=client, args=(range(t, len(jobs), 6),)) for t in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for (src, tgt), got in zip(jobs, results):
        want, _ = orc.translate_batch(src, tgt, kv_f16=True)
        assert got == want
    st = srv.stats()
    assert st["jobs"] == len(jobs) and st["sentences"] == sum(len(s) for s, _ in jobs)
    srv.stop()


def test_jobs_queued_behind_a_busy_gpu_share_batches(tiny):
    """While the first (large) job runs, the next ones queue up and are taken together:
    one group per (source, target, beam) key (server.rs:80-90)."""
    T, orc = tiny
    srv = M.Server(T)
    big = [pipeline_sentences()[i % 6] for i in range(32)]
    first = srv.submit(big, PLT, src_lang=254)
    jobs = _jobs(2, 12)
    handles = [srv.submit(src, tgt, src_lang=254) for src, tgt in jobs]
    assert first.result() == orc.translate_batch(big, PLT, kv_f16=True)[0]
    for (src, tgt), h in zip(jobs, handles):
        assert h.result() == orc.translate_batch(src, tgt, kv_f16=True)[0]
    st = srv.stats()
    assert st["jobs"] == 13 and st["groups"] < st["jobs"], st
    srv.stop()


def test_beam_and_greedy_jobs_group_separately(tiny):
    T, orc = tiny
    srv = M.Server(T, M.GenOptions(max_new_tokens=12))
    src = [s for s in pipeline_sentences() if len(s) == 9]  # one length: equal per-row budgets
    hb = [srv.submit(src, PLT, src_lang=254, beam_size=b) for b in (2, 1, 2, 1)]
    want_b, _ = orc.translate_batch(src, PLT, kv_f16=True, beam_size=2, max_new_tokens=12)
    want_g, _ = orc.translate_batch(src, PLT, kv_f16=True, max_new_tokens=12)
    assert [h.result() for h in hb] == [want_b, want_g, want_b, want_g]
    srv.stop()


def test_validation_and_stop_drains_the_queue(tiny):
    T, orc = tiny
    srv = M.Server(T)
    with pytest.raises(MalagaError):
        srv.submit([[254, 9999, 2]], PLT)
    with pytest.raises(MalagaError):
        srv.submit([[]], PLT)
    assert srv.submit([], PLT).result() == []
    jobs = _jobs(3, 6)
    handles = [srv.submit(src, tgt, src_lang=254) for src, tgt in jobs]
    srv.stop()  # finishes every queued job first
    for (src, tgt), h in zip(jobs, handles):
        assert h.done(0)
        assert h.result() == orc.translate_batch(src, tgt, kv_f16=True)[0]
