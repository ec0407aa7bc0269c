"""Known answers for the beam merge (src/translator.rs:250-335), worked out by hand from
the reference's rules, for both the oracle's merge (oracle.c beam_core, which its model
beam search runs) and the product's (BeamMerge, behind mlg_beam_search_host).  No GPU.

A scripted decoder replaces the model: each sentence maps the history of a decoder row
(the tokens fed after [decoder_start, tgt_lang], reordered with the row) to log-probs;
unlisted tokens, and unlisted histories entirely, get -20, so their top-2 are tokens 0
and 1 (ties go to the lowest index, translator.rs:343-358).  V = 6, EOS = 2, beam k = 2,
length penalty p = 1 unless stated: a finished hypothesis scores sum / (tokens + 1); all
numbers are dyadic, so every sum and quotient below is exact in f32.

Each case fixes the final tokens and the histories of every decoder row at every step
(the reorder and the fed tokens, including the padding rows: copies of beam 0 fed EOS,
translator.rs:312-317).  The last test plants one mistake at a time in the oracle and
checks that some case then fails, so none of these answers is vacuous for the rule it
is meant to pin.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

V, EOS, K = 6, 2, 2
INF = float("inf")

# ---------------------------------------------------------------------------- cases
# Each case: b sentences' scripts, max_new, penalty, expected result rows, expected row
# histories per step (step 1 first).  The traces are hand-worked from translator.rs.

CASE_A = dict(
    # Step 1: top-2 of [] is (3, -1), (EOS, -2): alive [3] (-1); done ([], -2/1 = -2);
    #   one done < k, no stop; pad row: old row 0 fed EOS.
    # Step 2: [3] -> (EOS, -1), (4, -2): candidates (-2, EOS), (-3, 4), pad row -inf ones.
    #   done ([3], -2/2 = -1); alive [3,4] (-3); the pad row's best (token 0, -inf) fills
    #   the second slot.  done = 2 >= k and best_done -1 >= best_alive -3/3 = -1 (equal):
    #   the sentence stops, and with it the search.  Result: [3].
    #   (With '>' instead of '>=' step 3 runs and [3,4,5] wins at -3.25/4.)
    scripts=[{(): {3: -1.0, 2: -2.0}, (3,): {2: -1.0, 4: -2.0}, (3, 4): {5: -0.25, 2: -0.5}}],
    max_new=3, p=1.0,
    result=[[3]],
    hist=[[(), ()], [(3,), (2,)]],
)

CASE_B = dict(
    # Step 1: (3, -1), (EOS, -1.25): alive [3] (-1); done ([], -1.25).
    # Step 2: [3] -> (4, -2), (EOS, -3): alive [3,4] (-3); done ([3], -4/2 = -2); pad
    #   row's token 0 alive at -inf.  best_done -1.25 < best_alive -3/3 = -1: go on.
    #   (penalty(step) instead of penalty(step + 1) gives -3/2 = -1.5 and stops with [].)
    # Step 3 = max_new: every candidate finishes: [3,4,5] -3.5/4 = -0.875, [3,4]
    #   -4/3, the pad row's two at -inf.  Result: [3,4,5].
    scripts=[{(): {3: -1.0, 2: -1.25}, (3,): {4: -2.0, 2: -3.0}, (3, 4): {5: -0.5, 2: -1.0}}],
    max_new=3, p=1.0,
    result=[[3, 4, 5]],
    hist=[[(), ()], [(3,), (2,)], [(3, 4), (2, 0)]],
)

CASE_C = dict(
    # Step 1: alive [3] (-1); done ([], -2).
    # Step 2 = max_new: [3] -> (4, -5), (EOS, -6): done [3,4] -6/3 = -2, [3] -7/2, and
    #   the pad row's [0], [1] at -inf.  Two finished hypotheses tie at -2: max_by keeps
    #   the last, [3,4] (the first would be []).
    scripts=[{(): {3: -1.0, 2: -2.0}, (3,): {4: -5.0, 2: -6.0}}],
    max_new=2, p=1.0,
    result=[[3, 4]],
    hist=[[(), ()], [(3,), (2,)]],
)

CASE_D = dict(
    # Step 1: (EOS, -0.5), (3, -1): done ([], -0.5); alive [3] (-1).  best_done -0.5 >=
    #   best_alive -1/2, but only one hypothesis is done (< k): go on.
    # Step 2: [3] -> (4, -0.25), (EOS, -0.5): alive [3,4] (-1.25); done ([3], -1.5/2).
    #   best_done -0.5 < -1.25/3: go on.  (penalty(step): -1.25/2 = -0.625, stops: [].)
    # Step 3: [3,4] -> (5, -0.125), (EOS, -0.25): [3,4,5] -1.375/4 = -0.34375 wins.
    scripts=[{(): {2: -0.5, 3: -1.0}, (3,): {4: -0.25, 2: -0.5}, (3, 4): {5: -0.125, 2: -0.25}}],
    max_new=3, p=1.0,
    result=[[3, 4, 5]],
    hist=[[(), ()], [(3,), (2,)], [(3, 4), (2, 0)]],
)

CASE_G = dict(
    # Step 1: alive [3] (-1); done ([], -2); pad row fed EOS: history (2,).
    # Step 2 = max_new: [3] -> (4, -1), (5, -2): [3,4] -2/3, [3,5] -3/3.  The pad row
    #   scripts strong tokens (5 at -0.125), but its hypothesis scores -inf, so [5] and
    #   [4] finish at -inf.  Result [3,4].  (A pad scored 0 would give [5] at -0.0625.)
    scripts=[{(): {3: -1.0, 2: -2.0}, (3,): {4: -1.0, 5: -2.0}, (2,): {5: -0.125, 4: -0.25}}],
    max_new=2, p=1.0,
    result=[[3, 4]],
    hist=[[(), ()], [(3,), (2,)]],
)

CASE_H = dict(
    # Two sentences: sentence 0 runs CASE_A's script and stops at step 2; sentence 1 runs
    # CASE_B's and goes on, so step 3 runs for both.  A stopped sentence keeps merging
    # (its rows still fill the batch) but records no more finished hypotheses: sentence 0
    # stays [3] although [3,4,5] (-0.8125) would beat it at step 3.  Rows 2, 3 belong to
    # sentence 1 (reorder indices offset by k).
    scripts=[CASE_A["scripts"][0], CASE_B["scripts"][0]],
    max_new=3, p=1.0,
    result=[[3], [3, 4, 5]],
    hist=[[(), (), (), ()], [(3,), (2,), (3,), (2,)], [(3, 4), (2, 0), (3, 4), (2, 0)]],
)

CASE_P2 = dict(
    # Length penalty p = 2: finished scores are sum / (tokens + 1)^2.
    # Step 1: (3, -1), (EOS, -3): alive [3]; done ([], -3/1).
    # Step 2 = max_new: [3] -> (4, -3), (EOS, -3.5): [3,4] -4/9 = -0.444, [3] -4.5/4;
    #   [3,4] wins.  With p = 0 (CASE_P0) nothing is normalized and [] wins at -3 over
    #   -4 and -4.5.
    scripts=[{(): {3: -1.0, 2: -3.0}, (3,): {4: -3.0, 2: -3.5}}],
    max_new=2, p=2.0,
    result=[[3, 4]],
    hist=[[(), ()], [(3,), (2,)]],
)

CASE_P0 = dict(CASE_P2, p=0.0, result=[[]])

CASES = dict(A=CASE_A, B=CASE_B, C=CASE_C, D=CASE_D, G=CASE_G, H=CASE_H, P2=CASE_P2, P0=CASE_P0)


def logprobs(case, row, hist):
    script = case["scripts"][row // K]
    out = np.full(V, -20.0, np.float32)
    for t, v in script.get(tuple(hist), {}).items():
        out[t] = v
    return out


def topk(row):
    order = sorted(range(V), key=lambda t: (-float(row[t]), t))[:K]
    return [float(row[t]) for t in order], order


# ------------------------------------------------------------------- runners

def run_oracle(case, mutant=0):
    import oracle as O

    L = O.lib()
    b = len(case["scripts"])
    seen = []

    @O.SCRIPT_FN
    def fn(_user, step, rows, hist, hist_len, out):
        h = [tuple(hist[r * hist_len + j] for j in range(hist_len)) for r in range(rows)]
        seen.append(h)
        for r in range(rows):
            lp = logprobs(case, r, h[r])
            for t in range(V):
                out[r * V + t] = float(lp[t])
        return 0

    res = np.zeros((b, max(case["max_new"], 1)), np.uint32)  # [b][max_new]
    n = np.zeros(b, np.int32)
    rc = L.orc_beam_scripted(b, K, V, EOS, case["max_new"], case["p"], 0, fn, None, mutant, res.ctypes.data,
                             n.ctypes.data)
    assert rc == 0
    return [res[i, : n[i]].tolist() for i in range(b)], seen


def run_product(case):
    from malaga_amd import _lib

    lib = _lib.load()
    b = len(case["scripts"])
    rows = b * K
    hist = [() for _ in range(rows)]
    seen, orders = [], []

    @_lib.BEAM_DECODE_FN
    def fn(_user, step, nrows, reorder, nxt, vals, idx):
        nonlocal hist
        assert nrows == rows
        if step > 1:
            ro, nx = [reorder[r] for r in range(rows)], [nxt[r] for r in range(rows)]
            orders.append((ro, nx))
            hist = [hist[ro[r]] + (nx[r],) for r in range(rows)]
        seen.append(list(hist))
        for r in range(rows):
            v, i = topk(logprobs(case, r, hist[r]))
            for j in range(K):
                vals[r * K + j] = v[j]
                idx[r * K + j] = i[j]
        return 0

    cap = case["max_new"] + 1
    out = np.zeros((b, cap), np.uint32)
    n = np.zeros(b, np.int32)
    _lib.check(lib.mlg_beam_search_host(b, K, case["max_new"], case["p"], EOS, fn, None, out.ctypes.data, cap,
                                        n.ctypes.data))
    return [out[i, : n[i]].tolist() for i in range(b)], seen, orders


# --------------------------------------------------------------------- tests

@pytest.mark.parametrize("name", list(CASES))
def test_oracle_known_answers(name):
    case = CASES[name]
    got, hist = run_oracle(case)
    assert got == case["result"]
    assert hist == case["hist"]


@pytest.mark.parametrize("name", list(CASES))
def test_product_known_answers(name):
    case = CASES[name]
    got, hist, _ = run_product(case)
    assert got == case["result"]
    assert hist == case["hist"]


def test_product_pads_continue_beam_zero():
    """The padding rows continue beam 0 of their sentence (translator.rs:314) and are fed
    EOS (315): CASE_H's step-1 merge pads row 1 from row 0 and row 3 from row 2."""
    _, _, orders = run_product(CASE_H)
    assert orders[0] == ([0, 0, 2, 2], [3, EOS, 3, EOS])
    assert orders[1] == ([0, 1, 2, 3], [4, 0, 4, 0])


# Mistakes planted in the oracle (oracle.c MUT_*) and a case each must fail.
MUTANTS = {1: "'>' instead of '>=' in the stop rule", 2: "best_alive / penalty(step)",
           3: "padding rows fed the pad id 1, not EOS", 4: "finished length = tokens, not tokens + 1",
           5: "first maximum in the final pick", 6: "stop without k finished hypotheses",
           8: "padding hypotheses scored 0, not -inf", 9: "stopped sentences keep finishing hypotheses"}


@pytest.mark.parametrize("mutant", list(MUTANTS))
def test_planted_mistakes_fail_a_known_answer(mutant):
    failed = []
    for name, case in CASES.items():
        got, hist = run_oracle(case, mutant)
        if got != case["result"] or hist != case["hist"]:
            failed.append(name)
    assert failed, f"no known answer catches: {MUTANTS[mutant]}"
