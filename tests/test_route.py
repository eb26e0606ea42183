"""CPU checks of the host routing (glmssd.moe.route, restating forward.rs:964-980) against an
independent brute-force selection, plus hand-computed cases: ordering by score + bias, the bias
only choosing (weights use the unbiased sigmoid scores), normalisation and scale, ties."""
import itertools

import numpy as np

from glmssd.moe import route


def brute(logits, bias, k, norm, scale):
    scores = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    best = max(itertools.combinations(range(len(bias)), k), key=lambda c: sum(scores[e] + bias[e] for e in c))
    best = sorted(best, key=lambda e: -(scores[e] + bias[e]))
    wsum = sum(scores[e] for e in best) if norm else 1.0
    return [(e, scores[e] / wsum * scale) for e in best]


def test_matches_brute_force():
    rng = np.random.default_rng(0)
    for trial in range(30):
        ne, k = 9, 3
        logits = rng.standard_normal((2, ne)).astype(np.float32) * 2
        bias = rng.standard_normal(ne).astype(np.float32) * 0.3
        norm, scale = bool(trial % 2), [1.0, 2.5][trial % 3 == 0]
        got = route(logits, bias, k, norm, scale)
        for t in range(2):
            want = brute(logits[t], bias, k, norm, scale)
            assert [e for e, _ in got[t]] == [e for e, _ in want]
            np.testing.assert_allclose([w for _, w in got[t]], [w for _, w in want], rtol=1e-6)


def test_hand_case():
    # scores sigmoid(0) = 0.5, sigmoid(2) ~ 0.8808, sigmoid(-2) ~ 0.1192; a bias of +1 on expert 2
    # makes it chosen first although its score is the lowest
    logits = np.array([[0.0, 2.0, -2.0, -5.0]], np.float32)
    bias = np.array([0.0, 0.0, 1.0, 0.0], np.float32)
    r = route(logits, bias, 2, True, 2.5)[0]
    assert [e for e, _ in r] == [2, 1]
    s2, s1 = 1 / (1 + np.exp(2.0)), 1 / (1 + np.exp(-2.0))
    np.testing.assert_allclose([w for _, w in r], [s2 / (s1 + s2) * 2.5, s1 / (s1 + s2) * 2.5], rtol=1e-6)
    # without normalisation the weights are the scaled scores
    r = route(logits, bias, 2, False, 1.0)[0]
    np.testing.assert_allclose([w for _, w in r], [s2, s1], rtol=1e-6)


def test_ties_keep_id_order():
    r = route(np.zeros((1, 5), np.float32), np.zeros(5, np.float32), 3)[0]
    assert [e for e, _ in r] == [0, 1, 2]
    np.testing.assert_allclose([w for _, w in r], [1 / 3] * 3, rtol=1e-6)


def test_slot_index_is_rank_times_tokens_plus_token():
    """forward.rs:1039-1048: slot = (rank of the expert in the token's route) * t + token; the
    slots of all pairs are exactly 0 .. k*t-1 (each (rank, token) once)."""
    from glmssd.moe import group_pairs, slot_index
    rng = np.random.default_rng(5)
    t, ne, k = 7, 12, 4
    routes = [[(int(e), float(rng.random())) for e in rng.permutation(ne)[:k]] for _ in range(t)]
    offs, idx, w, pe = group_pairs(routes, ne)
    sl = slot_index(routes, idx, pe)
    assert sorted(sl.tolist()) == list(range(k * t))
    for p in range(idx.size):
        ti, e = int(idx[p]), int(pe[p])
        assert routes[ti][sl[p] // t][0] == e and sl[p] % t == ti
        assert routes[ti][sl[p] // t][1] == w[p]
