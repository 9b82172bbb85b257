"""Pin the CPU oracle: golden vectors from the reference's own comparator,
known-answer tests, exhaustive enumeration, float64 optima, status rules and
optimized-mode cases whose diagnostics follow from the reference's rules."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import collapse, dp_optimum, exhaustive_best, golden_cases, split
from oracle import oracle as O


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: c[0])
def test_golden_vectors_bit_exact(case):
    name, e, y, blank, labels, scores = case
    out = O.align([e], [y], blank_id=blank, mode="conventional")
    assert out["status"].tolist() == [0]
    np.testing.assert_array_equal(out["labels"], labels)
    np.testing.assert_array_equal(out["scores"].view(np.int32), scores.view(np.int32))


def test_golden_vectors_pin_the_tie_rule():
    """A Viterbi whose ties prefer advance over stay (the rule the reference
    corrected, benchmarks/patches/README.md) disagrees with the golden vectors;
    the reference rule reproduces all of them."""
    def viterbi(e, y, blank, prefer_advance):
        S = 2 * len(y) + 1
        lab = np.full(S, blank); lab[1::2] = y
        a = np.full(S, -np.inf, np.float32); a[:2] = e[0, lab[:2]]
        bp = np.zeros((len(e), S), np.int8)
        for t in range(1, len(e)):
            n = np.empty_like(a)
            for s in range(S):
                cand = [(a[s], 0)]
                if s >= 1: cand.append((a[s - 1], 1))
                if s >= 2 and lab[s] != blank and lab[s] != lab[s - 2]: cand.append((a[s - 2], 2))
                best, j = cand[0]
                for v, jj in cand[1:]:
                    if v > best or (prefer_advance and v == best):
                        best, j = v, jj
                n[s] = np.float32(best + e[t, lab[s]]); bp[t, s] = j
            a = n
        s = S - 1 if not (S > 1 and a[S - 2] >= a[S - 1]) else S - 2
        path = []
        for t in range(len(e) - 1, -1, -1):
            path.append(lab[s]); s -= bp[t, s]
        return np.array(path[::-1])
    cases = [c for c in golden_cases() if c[0].startswith(("ties", "tie", "adapters"))]
    right = sum(np.array_equal(viterbi(e, y, b, False), lab) for _, e, y, b, lab, _ in cases)
    wrong = sum(np.array_equal(viterbi(e, y, b, True), lab) for _, e, y, b, lab, _ in cases)
    assert right == len(cases)
    assert wrong < len(cases)


def test_compiled_reference_agrees_on_random_inputs():
    ref = O.reference_comparator()
    if ref is None:
        pytest.skip("oracle/_ref is built only where the reference tree is mounted")
    rng = np.random.default_rng(7)
    for trial in range(150):
        V = int(rng.integers(3, 40))
        blank = int(rng.integers(0, V))
        vocab = [v for v in range(V) if v != blank]
        y = rng.choice(vocab, int(rng.integers(1, 30))).astype(np.int64)
        R = int((y[1:] == y[:-1]).sum())
        T = int(rng.integers(y.size + R + 2, y.size + R + 150))
        e = (rng.integers(-3, 0, (T, V)) if trial % 3 == 0 else np.log(rng.dirichlet(np.ones(V), T))).astype(np.float32)
        lab, sc = ref.forced_align(e[None], y[None], blank)
        out = O.align([e], [y], blank_id=blank, mode="conventional")
        np.testing.assert_array_equal(out["labels"], np.asarray(lab).reshape(-1))
        np.testing.assert_array_equal(out["scores"], np.asarray(sc).reshape(-1))


def test_known_answers():
    # predecessor-tie case (benchmarks/tests/test_adapters.py:55-68): corrected score 0
    e = np.array([[0, 0, -10], [0, 0, -10], [-10, -10, 0], [0, -10, -10], [0, -10, -10]], np.float32)
    out = O.align([e], [np.array([1, 2])], mode="conventional")
    assert out["labels"].tolist() == [1, 0, 2, 0, 0]
    assert out["scores"].sum() == 0
    # examples/align_emissions.py:5-14: per-frame argmax is a legal path
    x = np.array([[0., -4., -4.], [-4., 0., -4.], [0., -4., -4.],
                  [-4., 0., -4.], [-4., -4., 0.], [0., -4., -4.]], np.float32)
    e = (x - np.log(np.exp(x).sum(1, keepdims=True))).astype(np.float32)
    for mode in ("optimized", "conventional"):
        assert O.align([e], [np.array([1, 1, 2])], mode=mode)["labels"].tolist() == [0, 1, 0, 1, 2, 0]
    # label fixtures of benchmarks/tests/test_adapters.py:19-31
    for labels, targets, blank in (([0, 1, 1, 0, 2, 2], [1, 2], 0), ([3, 0, 0, 3, 0, 2, 3], [0, 0, 2], 3),
                                   ([0, 1, 0, 1, 2, 0, 0, 0], [1, 1, 2], 0)):
        e = np.full((len(labels), 4), -8, dtype=np.float32)
        e[np.arange(len(labels)), labels] = -0.125
        for mode in ("optimized", "conventional"):
            assert O.align([e], [np.array(targets)], blank_id=blank, mode=mode)["labels"].tolist() == labels


@pytest.mark.parametrize("tokens", [1, 2, 5, 64])
def test_tight_frames_closed_form(tokens):
    """All-equal tokens with T = 2U - 1 admit one path: token, blank, token, ...
    (tests/test_async_validation.py:39-56)."""
    y = np.ones(tokens, np.int64)
    e = np.zeros((2 * tokens - 1, 3), np.float32)
    for mode in ("optimized", "conventional"):
        out = O.align([e, e[:-1]] if tokens > 1 else [e], [y, y] if tokens > 1 else [y], mode=mode)
        assert out["labels"][: 2 * tokens - 1].tolist() == [1 if i % 2 == 0 else 0 for i in range(2 * tokens - 1)]
        assert out["status"].tolist() == ([0, 4] if tokens > 1 else [0])


def test_exhaustive_enumeration_small():
    """Oracle path scores equal the best legal path found by enumeration
    (pattern of benchmarks/tests/test_adapters.py:236-270)."""
    rng = np.random.default_rng(1729)
    for index in range(12):
        blank = index % 3
        vocab = [v for v in range(3) if v != blank]
        y = np.array([vocab[index % 2], vocab[(index // 2) % 2]], np.int64)
        T = 5 + index % 2
        e = rng.integers(-5, 1, size=(T, 3)).astype(np.float32)
        best = exhaustive_best(e, y, blank)
        for mode in ("optimized", "conventional"):
            out = O.align([e], [y], blank_id=blank, mode=mode)
            assert collapse(out["labels"], blank).tolist() == y.tolist()
            assert float(out["scores"].astype(np.float64).sum()) == best


@pytest.mark.parametrize("blank", [0, 5])
def test_float64_optimum_on_integer_emissions(blank):
    """tests/test_core.py:31-48: ragged integer emissions, exact float64 optimum."""
    rng = np.random.default_rng(32)
    labels = np.array([i for i in range(6) if i != blank])
    values = [rng.integers(-9, 0, (n, 6)).astype(np.float32) for n in (7, 129, 257, 2305)]
    tokens = [rng.choice(labels, n) for n in (0, 11, 44, 120)]
    for mode in ("optimized", "conventional"):
        out = O.align(values, tokens, blank_id=blank, mode=mode)
        assert out["status"].tolist() == [0, 0, 0, 0]
        for v, t, p, s in zip(values, tokens, split(out["labels"], out["lengths"]), split(out["scores"], out["lengths"])):
            assert collapse(p, blank).tolist() == t.tolist()
            np.testing.assert_array_equal(s, v[np.arange(len(p)), p])
            assert s.astype(np.float64).sum() == dp_optimum(v, t, blank)


def test_status_rules():
    """Exact status vectors of tests/test_async_validation.py and
    tests/test_emission_validity.py."""
    e = np.log(np.random.default_rng(12).dirichlet(np.ones(6), 257)).astype(np.float32)
    token_lists = [[1, 1, 2], [-1], [6], [0], [2**32 + 1], [2**63 - 1], [-2**63], []]
    for mode in ("optimized", "conventional"):
        out = O.align([e] * 8, [np.array(t, np.int64) for t in token_lists], mode=mode)
        assert out["status"].tolist() == [0, 3, 3, 3, 3, 3, 3, 0]
        emissions = [np.zeros((3, 4), np.float32) for _ in range(5)]
        emissions[-1][:] = -np.inf
        out = O.align(emissions, [np.array(t) for t in ([9], [1, 1, 1], [1], [0, 0, 0, 0], [1])], mode=mode,
                      emission_validity=np.array([False, False, False, True, True]))
        assert out["status"].tolist() == [3, 4, 2, 3, 1]
        assert (out["labels"] == -1).all() and np.isneginf(out["scores"]).all()
        assert np.isneginf(out["objective"]).all()
    # in-vocabulary but infeasible: 4 when checked, 1 (no finite path) unchecked
    e = np.zeros((2, 4), np.float32)
    assert O.align([e], [np.array([1, 1])])["status"].tolist() == [4]
    assert O.align([e], [np.array([1, 1])], check_inputs=False)["status"].tolist() == [1]


def _chunk_objective(scores, H=128):
    """Optimized-mode objective: fp32 sequential sum inside each chunk, then an
    fp32 sum of chunk results in order (alignment.cu:135-137, 583)."""
    total = np.float32(0)
    for a in range(0, len(scores), H):
        acc = np.float32(scores[a])
        for v in scores[a + 1:a + H]:
            acc = np.float32(acc + v)
        total = np.float32(total + acc)
    return total


def test_optimized_peaky_shortcuts_and_objective():
    from fast_forced_aligner import workloads as W
    rng = np.random.default_rng(3)
    es, ys = [], []
    for T in (130, 700, 1000):
        y = rng.integers(1, 32, size=T // 4).astype(np.int64)
        es.append(W.peaky(rng, y, T, 32))
        ys.append(y)
    conv = O.align(es, ys, mode="conventional")
    opt = O.align(es, ys, mode="optimized")
    np.testing.assert_array_equal(opt["labels"], conv["labels"])
    np.testing.assert_array_equal(opt["scores"], conv["scores"])
    assert opt["stitched"].tolist() == [1, 1, 1]
    n = [(len(e) + 127) // 128 for e in es]
    assert opt["shortcut_stats"].tolist() == [[k, len(e), 0] for k, e in zip(n, es)]
    for s, obj in zip(split(opt["scores"], opt["lengths"]), opt["objective"]):
        assert _chunk_objective(s).view(np.int32) == np.float32(obj).view(np.int32)
    assert opt["reuse_stats"].shape == (0, 4) and conv["reuse_stats"].shape == (0, 4)
    assert not conv["stitched"].any() and not conv["shortcut_stats"].any()


def test_optimized_ambiguous_blank_chunk():
    """A middle chunk whose greedy path is all blank has L+1 placements: it is
    counted as ambiguous (shortcut_stats[2]) and solved by chunk DP."""
    T, V = 384, 8
    labels = np.zeros(T, np.int64)
    labels[10:20] = 1
    labels[300:310] = 2
    e = np.full((T, V), -6.0, np.float32)
    e[np.arange(T), labels] = -0.01
    out = O.align([e], [np.array([1, 2])], mode="optimized")
    conv = O.align([e], [np.array([1, 2])], mode="conventional")
    assert out["shortcut_stats"].tolist() == [[2, 256, 1]]
    np.testing.assert_array_equal(out["labels"], conv["labels"])
    assert out["stitched"].tolist() == [1]


def test_optimized_long_record_early_fallback():
    """T >= 2048 enables the 512-frame repair budget (alignment.cu:175-198): a
    900-frame noisy region breaks every seam inside it, the proposed repair
    spans more than 512 frames, so the record takes the early full fallback
    (routing state 2) and equals conventional DP."""
    from fast_forced_aligner import workloads as W
    rng = np.random.default_rng(11)
    T = 2305
    y = rng.integers(1, 32, size=600).astype(np.int64)
    e = W.peaky(rng, y, T, 32)
    e[700:1600] = W._log_softmax(3 * rng.standard_normal((900, 32)).astype(np.float32))
    opt = O.align([e], [y], mode="optimized")
    conv = O.align([e], [y], mode="conventional")
    np.testing.assert_array_equal(opt["labels"], conv["labels"])
    assert opt["routing_stats"][0, 0] == 2 and opt["routing_stats"][0, 1] == 1
    assert opt["routing_stats"][0, 2] > 512
    assert opt["stitched"].tolist() == [0] and opt["repair_passes"].tolist() == [0]
    # every DP chunk wrote its S-value frontier; chunk 0 was a shortcut, so no resume
    dp_chunks = 19 - opt["shortcut_stats"][0, 0]
    assert opt["reuse_stats"].tolist() == [[0, 0, dp_chunks * 1201, 0]]


def test_empty_targets_all_blank():
    e = np.log(np.random.default_rng(0).dirichlet(np.ones(4), 300)).astype(np.float32)
    for mode in ("optimized", "conventional"):
        out = O.align([e], [np.array([], np.int64)], mode=mode)
        assert out["status"].tolist() == [0]
        assert (out["labels"] == 0).all()


def test_emission_valid():
    e = np.zeros((5, 4), np.float32)
    assert O.emission_valid(e)
    e[2, 1] = -np.inf
    assert O.emission_valid(e)
    e[3, 0] = np.nan
    assert not O.emission_valid(e)
    e[3, 0] = np.inf
    assert not O.emission_valid(e)


# --- optimized-mode repair rounds, budget and frontier: hand-derived pins ---

import repair_cases as RC  # noqa: E402


@pytest.mark.parametrize("case", RC.all_cases(), ids=lambda c: c["name"])
def test_repair_path_hand_derived(case):
    """Merges, repair passes, repaired frames, frontier resume columns, budget
    rejection with and without overlap, and the repair_rounds / mode knobs:
    every output equals the values derived on paper from alignment.cu in
    tests/repair_cases.py, and the labels equal conventional DP."""
    knobs = RC.knob_vector(**case["knobs"])
    out = O.align([case["emissions"]], [case["targets"]], options=RC.oracle_options(knobs))
    RC.check_expected(out, case)
    conv = O.align([case["emissions"]], [case["targets"]], mode="conventional")
    np.testing.assert_array_equal(out["labels"], conv["labels"])


# Planted mistakes (oracle/ffa_oracle.c MUT(n), compiled only into the
# mutants library): each is a plausible misreading of alignment.cu, and each
# must make at least one hand-derived case fail.
PLANTED = {
    1: "strict start at every chunk (no relaxed init for a > 0, cu:409)",
    2: "chunk terminal takes the highest index on ties (cu:462-492)",
    3: "budget compared against twice the budget (cu:190-192)",
    4: "routing_stats[1] set once instead of counted per round (cu:194)",
    5: "merge pass checks seams against the group's end, not the previous piece's (cu:206-219)",
    6: "repaired_frames counts every interval, not only merged ones (cu:222-226)",
    7: "frontier resume counts the saved end, not the resumed frames (cu:378)",
    8: "the full fallback also counts written frontier values (cu:381)",
    9: "legal_seam accepts every jump of two (cu:157-161)",
}


@pytest.mark.parametrize("mistake", sorted(PLANTED), ids=lambda n: f"mut{n}")
def test_repair_pins_reject_planted_mistakes(mistake):
    lib = O.mutants()
    failures = 0
    try:
        lib.orc_set_mutant(mistake)
        for case in RC.all_cases():
            out = O.align([case["emissions"]], [case["targets"]],
                          options=RC.oracle_options(RC.knob_vector(**case["knobs"])), library=lib)
            try:
                RC.check_expected(out, case)
            except AssertionError:
                failures += 1
    finally:
        lib.orc_set_mutant(0)
    assert failures > 0, f"no pin rejects: {PLANTED[mistake]}"


def test_mutants_library_is_the_oracle_when_no_mistake_is_planted():
    lib = O.mutants()
    lib.orc_set_mutant(0)
    for case in RC.all_cases():
        out = O.align([case["emissions"]], [case["targets"]],
                      options=RC.oracle_options(RC.knob_vector(**case["knobs"])), library=lib)
        RC.check_expected(out, case)
