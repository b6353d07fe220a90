"""Pins oracle/lookup.py against the reference's hand-traced known answers
(tests/test_lookup_acceptance.py:7-27, fixture tests/golden/lookup_known_answers.json) and the
brute-force equivalence the reference tests demand of its index (tests/test_dflash.py:90-123)."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import lookup as O

GOLD = json.loads((Path(__file__).parent / "golden" / "lookup_known_answers.json").read_text())


def ref_sequences():
    return [
        [int(t) for t in np.random.default_rng(1).integers(0, 5, size=300)],
        [int(t) for t in np.random.default_rng(2).integers(0, 1000, size=300)],
        [1, 2, 3, 4, 5] * 20 + [1, 2, 9] * 10 + [7] * 30,
    ]


def test_lookup_known_answers():
    for c in GOLD["cases"]:
        assert O.lookup(GOLD["ids"], c["t"], c["g"], c["n"]) == c["want"]


def test_boundary_known_answer():
    ids = GOLD["ids_boundary"]
    c = GOLD["boundary_case"]
    d = O.lookup(ids, c["t"], c["g"], c["n"])
    win = ids[c["t"]:c["t"] + len(d)]
    k = 0
    while k < min(len(d), len(win)) and d[k] == win[k]:
        k += 1
    assert k == c["common_prefix_with_ids_from_t"]


@pytest.mark.parametrize("g", [1, 2, 3, 4])
def test_dict_index_and_scan_match_lookup_on_known_ids(g):
    ids = GOLD["ids"]
    idx = O.DictIndex(g)
    for t in range(len(ids) + 1):
        want = O.lookup(ids, t, g, 15)
        assert idx.propose(15) == want
        cnt, pos, got = O.propose_scan(np.array(ids, np.int32), t, g, 15)
        assert got == want and cnt == len(want)
        if t < len(ids):
            idx.extend(ids[t:t + 1])


@pytest.mark.parametrize("seq_i", [0, 1, 2])
@pytest.mark.parametrize("g", [1, 3, 4])
def test_matches_brute_force_exhaustively(seq_i, g):
    seq = ref_sequences()[seq_i]
    h = np.array(seq, np.int32)
    idx = O.DictIndex(g)
    for t in range(len(seq) + 1):
        for n in (1, 7, 15):
            want = O.lookup(seq, t, g, n)
            assert idx.propose(n) == want, (t, n)
            cnt, pos, got = O.propose_scan(h, t, g, n)
            assert got == want, (t, n)
            if want:
                # pos is the most recent earlier start: hist[pos:pos+g] == last g ids
                assert seq[pos:pos + g] == seq[t - g:t] and pos <= t - g - 1
        if t < len(seq):
            idx.extend(seq[t:t + 1])


def test_bulk_extend_matches_incremental():
    seq = [int(t) for t in np.random.default_rng(3).integers(0, 4, size=200)]
    a, b = O.DictIndex(3), O.DictIndex(3)
    a.extend(seq)
    for i in range(0, 200, 7):
        b.extend(seq[i:i + 7])
    assert a.last == b.last and a.propose(15) == b.propose(15) == O.lookup(seq, 200, 3, 15)


def test_overlapping_match_and_truncation():
    # [7]*6: key (7,7,7) at t=6, most recent earlier start s = t-g-1 = 2; continuation ids[5:6]
    seq = [7] * 6
    assert O.lookup(seq, 6, 3, 4) == [7]
    assert O.propose_scan(np.array(seq, np.int32), 6, 3, 4) == (1, 2, [7])


def test_most_recent_match_wins():
    seq = [1, 2, 3, 10, 1, 2, 3, 20, 5, 1, 2, 3]
    assert O.lookup(seq, len(seq), 3, 4) == [20, 5, 1, 2]
    assert O.propose_scan(np.array(seq, np.int32), len(seq), 3, 4)[1] == 4


def test_greedy_accept_cases():
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((5, 50)).astype(np.float32)
    pred = logits.argmax(-1)
    for m in range(5):
        drafts = list(pred[:m]) + [int(pred[m]) + 1] * (4 - m)  # first mismatch at slot m
        k, nxt = O.greedy_accept(logits, drafts)
        assert k == m and nxt == int(pred[m])
    k, nxt = O.greedy_accept(logits, list(pred[:4]))
    assert k == 4 and nxt == int(pred[4])
    assert O.greedy_accept(logits, []) == (0, int(pred[0]))


def test_greedy_accept_ties_take_first_index():
    logits = np.zeros((2, 8), np.float32)
    logits[0, [3, 5]] = 1.0
    logits[1, [0, 7]] = 2.0
    assert O.greedy_accept(logits, [3]) == (1, 0)
    assert O.greedy_accept(logits, [5]) == (0, 3)


def test_planted_off_by_one_is_caught():
    # allowing the gram to match itself (s <= t-g) must break the known answers
    def bad(ids, t, g, n):
        if t < g:
            return []
        key = tuple(ids[t - g:t])
        for s in range(t - g, -1, -1):
            if tuple(ids[s:s + g]) == key:
                return list(ids[s + g:min(s + g + n, t)])
        return []

    assert any(bad(GOLD["ids"], c["t"], c["g"], c["n"]) != c["want"] for c in GOLD["cases"])
