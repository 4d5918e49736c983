"""Pin the CPU oracle's acceptance restatement (candidates, verify, merge, RNG).

Independent checks: the reference's own known-answer tests
(tests/ops/test_cuda_speculative.py, tests/generation/test_tp_sampling.py),
a double-precision dictionary model of p/q rejection sampling written here,
the Random123 Philox4x32-10 vectors, libm expf, and brute-force sorting.
"""
from __future__ import annotations

import math
import random

import numpy as np
import pytest

NAN_BF16 = np.uint16(0x7FC0)


def bf16(values):
    from oracle import oracle as o
    return o.f32_to_bf16_bits(np.asarray(values, np.float32))


# --------------------------------------------------------------------------- #
# RNG and exp
# --------------------------------------------------------------------------- #
def test_philox_random123_known_answers(oracle):
    assert oracle.philox4x32_10([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert oracle.philox4x32_10([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [
        0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert oracle.philox4x32_10([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
                                [0xA4093822, 0x299F31D0]) == [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_philox_uniform_maps_first_word_like_tl_rand(oracle):
    for seed, ordinal in ((0, 0), (7, 3), (2**40 + 5, 11), (123456789, 2**31 + 9)):
        word = oracle.philox4x32_10([ordinal & 0xFFFFFFFF, 0, 0, 0],
                                    [seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF])[0]
        signed = word - 2**32 if word >= 2**31 else word
        signed = -signed - 1 if signed < 0 else signed
        want = float(np.float32(np.float32(signed) * np.float32(4.6566127342e-10)))
        assert oracle.philox_uniform(seed, ordinal) == want
        assert 0.0 <= want < 1.0


def test_expf_within_two_ulp_of_libm(oracle):
    xs = np.concatenate([np.linspace(-103.0, 88.7, 200001, dtype=np.float32),
                         np.linspace(-1.0, 0.0, 50001, dtype=np.float32),
                         np.array([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30], np.float32)])
    worst = 0
    for x in xs.tolist():
        got = np.float32(oracle.expf(x))
        want = np.float32(math.exp(float(np.float32(x))))  # exact to double, rounded once
        if want == 0 or not np.isfinite(want):
            continue
        ulps = abs(int(got.view(np.int32)) - int(want.view(np.int32)))
        worst = max(worst, ulps)
    assert worst <= 2, worst
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(float("-inf")) == 0.0
    assert math.isinf(oracle.expf(89.0))


# --------------------------------------------------------------------------- #
# Candidate preparation
# --------------------------------------------------------------------------- #
def test_candidates_match_brute_force_sort(oracle):
    rng = np.random.default_rng(11)
    rows, width, count = 6, 300, 20
    values = np.round(rng.standard_normal((rows, width)) * 4) / 4  # many exact ties
    logits = bf16(values)
    logits[2, 17] = np.uint16(0x8000)  # -0.0 ties with +0.0 by value
    temps = np.array([0.7, 0.0, 1.0, 0.0, 0.5, 1.0], np.float32)
    logits[5, 123] = np.uint16(0x7F80)  # +inf: non-finite row
    scores, ids = oracle.candidates(logits, temps, count, capacity=24, owned_rows=5)
    f = oracle.bf16_bits_to_f32(logits)
    for r in range(rows):
        if r >= 5:
            assert (ids[r] == -1).all() and (scores[r] == NAN_BF16).all()
            continue
        order = sorted(range(width), key=lambda j: (-float(f[r, j]), j))
        if temps[r] == 0:
            assert ids[r, 0] == order[0] and scores[r, 0] == logits[r, order[0]]
            assert (ids[r, 1:] == -1).all()
        else:
            assert ids[r, :count].tolist() == order[:count]
            assert scores[r, :count].tolist() == logits[r, order[:count]].tolist()
            assert (ids[r, count:] == -1).all()
    # non-finite owned row publishes id -2 in every counted slot
    logits[1, 3] = np.uint16(0x7FC0)
    _, ids = oracle.candidates(logits, temps, count, capacity=24, owned_rows=6)
    assert (ids[1, :count] == -2).all() and (ids[1, count:] == -1).all()
    assert (ids[5, :count] == -2).all()


def test_fp16_candidates_match_brute_force_sort(oracle):
    """fp16 logits (local_candidates.py:41 admits them): same order by value
    with ascending ids on ties, fp16 scores published unchanged, fp16 NaN padding."""
    rng = np.random.default_rng(12)
    rows, width, count = 5, 300, 20
    values = (np.round(rng.standard_normal((rows, width)) * 4) / 4).astype(np.float16)
    logits = values.view(np.uint16).copy()
    logits[2, 17] = np.uint16(0x8000)          # -0.0 ties with +0.0
    logits[3, 5] = np.uint16(0x0001)           # smallest subnormal
    temps = np.array([0.7, 0.0, 1.0, 0.5, 1.0], np.float32)
    logits[4, 200] = np.uint16(0xFC00)         # -inf: non-finite row
    scores, ids = oracle.candidates(logits, temps, count, capacity=24, fp16=True)
    f = logits.view(np.float16).astype(np.float64)
    for r in range(rows):
        if r == 4:
            assert (ids[r, :count] == -2).all() and (scores[r] == 0x7E00).all()
            continue
        order = sorted(range(width), key=lambda j: (-f[r, j], j))
        if temps[r] == 0:
            assert ids[r, 0] == order[0] and scores[r, 0] == logits[r, order[0]]
            assert (ids[r, 1:] == -1).all() and (scores[r, 1:] == 0x7E00).all()
        else:
            assert ids[r, :count].tolist() == order[:count]
            assert scores[r, :count].tolist() == logits[r, order[:count]].tolist()
    # the same values as bf16 bits order differently only through rounding:
    # exact fp16 -> bf16 conversion of quarter-integers keeps the order
    bf = bf16(values.astype(np.float32))
    s2, i2 = oracle.candidates(bf[:4], temps[:4], count, capacity=24)
    assert (i2 == ids[:4]).all()


def test_f32_candidates_match_brute_force_sort(oracle):
    """fp32 logits (local_candidates.py:41, SCORE_TYPE 2): order by float32 value
    with ascending ids on ties (-0 == +0), scores published bit for bit, fp32 NaN
    padding, -2 for rows with a non-finite logit; all_random greedy rows pad."""
    rng = np.random.default_rng(13)
    rows, width, count = 6, 300, 20
    logits = (np.round(rng.standard_normal((rows, width)) * 4) / 4).astype(np.float32)
    logits[0, 40] = logits[0, 260] = 9.0                    # tie for the maximum
    logits[2] = -np.abs(logits[2]) - 1.0
    logits[2, 17], logits[2, 9] = np.float32(-0.0), np.float32(0.0)  # -0 ties with +0
    logits[3, 5] = np.float32(1.4e-45)                         # smallest subnormal
    logits[3, 6] = np.float32(np.nextafter(np.float32(0.25), np.float32(1)))  # one ulp above a tie
    logits[5, 123] = -np.inf
    temps = np.array([0.7, 0.0, 0.0, 1.0, 0.5, 1.0], np.float32)
    scores, ids = oracle.candidates_f32(logits, temps, count, capacity=24)
    bits = logits.view(np.uint32)
    nan_bits = np.uint32(0x7FC00000)
    for r in range(rows):
        got = scores[r].view(np.uint32)
        if r == 5:
            assert (ids[r, :count] == -2).all() and (ids[r, count:] == -1).all()
            assert (got == nan_bits).all()
            continue
        order = sorted(range(width), key=lambda j: (-float(logits[r, j]), j))
        if temps[r] == 0:
            assert ids[r, 0] == order[0] and got[0] == bits[r, order[0]]
            assert (ids[r, 1:] == -1).all() and (got[1:] == nan_bits).all()
        else:
            assert ids[r, :count].tolist() == order[:count]
            assert got[:count].tolist() == bits[r, order[:count]].tolist()
            assert (ids[r, count:] == -1).all()
    assert ids[0, 0] == 40 and ids[2, 0] == 9 and scores[2, 0].view(np.uint32) == 0  # +0 at id 9 first
    # all_random: greedy rows publish padding; owned_rows pads the rest
    s2, i2 = oracle.candidates_f32(logits, temps, count, capacity=24, all_random=True, owned_rows=4)
    assert (i2[1] == -1).all() and (i2[2] == -1).all() and (i2[4:] == -1).all()
    assert (i2[0] == ids[0]).all() and (i2[3] == ids[3]).all()
    # the bf16 restatement agrees where the values are exact in bf16
    b, bi = oracle.candidates(bf16(logits[:1]), temps[:1], count, capacity=24)
    assert (bi == ids[:1]).all()


# --------------------------------------------------------------------------- #
# verify_k1: reference known answers
# --------------------------------------------------------------------------- #
def _full(shape, value, dtype):
    return np.full(shape, value, dtype)


def test_grammar_underfill_never_relaxes_unconstrained_request_guard(oracle):
    # tests/ops/test_cuda_speculative.py:73-100
    scores = _full((1, 2, 20), NAN_BF16, np.uint16)
    ids = _full((1, 2, 20), -1, np.int64)
    target = _full((1, 4, 20), NAN_BF16, np.uint16)
    target_ids = _full((1, 4, 20), -1, np.int64)
    scores[:, :, 0] = target[:, :, 0] = bf16([1.0])[0]
    ids[:, :, 0] = target_ids[:, :, 0] = 3
    dec = oracle.verify_k1(scores, ids, target, target_ids, [0, 2], [3, 3], [1.0, 1.0], [1.0, 1.0],
                           [20, 20], [1, 1], [0, 0], 2, uniforms=[[0.5, 0.5], [0.5, 0.5]],
                           allow_underfilled=True, constrained_rows=[True, False])
    assert dec.tolist() == [[1, 3], [-1, -1]]


@pytest.mark.parametrize("source", ["q", "p0", "p1"])
@pytest.mark.parametrize("score,token", [(math.nan, -2), (math.nan, 9), (math.inf, 9), (-math.inf, 9)])
def test_owned_failure_is_not_padding_when_other_shards_supply_topk(oracle, source, score, token):
    # tests/ops/test_cuda_speculative.py:102-131
    q = _full((4, 4, 20), NAN_BF16, np.uint16)
    qi = _full((4, 4, 20), -1, np.int64)
    p = _full((4, 8, 20), NAN_BF16, np.uint16)
    pi = _full((4, 8, 20), -1, np.int64)
    q[0, :3, 0], qi[0, :3, 0] = bf16([2.0])[0], 10
    p[0, :, 0] = bf16([2.0])[0]
    pi[0, ::2, 0], pi[0, 1::2, 0] = 10, 11
    physical_rows = (4, 2, 0)
    s, i, row = (q, qi, 1) if source == "q" else (p, pi, physical_rows[1] + (source == "p1"))
    s[3, row, 0], i[3, row, 0] = bf16([score])[0], token
    dec = oracle.verify_k1(q, qi, p, pi, (*physical_rows, 0), [10] * 4, [1.0] * 4, [1.0] * 4,
                           [1] * 4, [1] * 4, [0] * 4, 3, uniforms=np.full((4, 2), 0.5))
    assert dec.tolist() == [[1, 11], [-1, -1], [1, 11], [-1, -1]]


def _distribution(pairs, temperature):
    """Double-precision sorted-candidate softmax (independent dictionary model)."""
    ordered = sorted(pairs, key=lambda item: (-item[0], item[1]))
    if temperature == 0.0:
        return {ordered[0][1]: 1.0}
    top = ordered[0][0] / temperature
    weights = [math.exp(score / temperature - top) for score, _ in ordered]
    total = sum(weights)
    return {tok: w / total for w, (_, tok) in zip(weights, ordered)}


def _draw(probabilities, uniform):
    cumulative = 0.0
    for tok, prob in probabilities.items():
        cumulative += prob
        if cumulative > uniform:
            return tok
    raise AssertionError("uniform outside mass")


def _dict_oracle(q, p0, p1, draft, temperature, u_accept, u_sample):
    qd, p0d, p1d = (_distribution(x, temperature) for x in (q, p0, p1))
    if temperature == 0.0:
        accepted = draft == next(iter(p0d))
    else:
        accepted = u_accept < min(1.0, p0d.get(draft, 0.0) / qd[draft])
    if accepted:
        return 1, _draw(p1d, u_sample)
    residual = {t: max(0.0, p0d.get(t, 0.0) - qd.get(t, 0.0)) for t in p0d.keys() | qd.keys()}
    mass = sum(residual.values())
    # the device kernel walks the residual in p0's candidate order
    ordered = {t: residual[t] / mass for t in p0d if residual.get(t, 0.0) > 0.0}
    return 0, _draw(ordered, u_sample)


def test_k1_decisions_match_independent_dictionary_model(oracle):
    # tests/ops/test_cuda_speculative.py:230-309 (TP=4, two ranks populated)
    tp, rows, k, p_rows = 4, 4, 20, 8
    q_s = _full((tp, rows, k), NAN_BF16, np.uint16)
    q_i = _full((tp, rows, k), -1, np.int64)
    p_s = _full((tp, p_rows, k), NAN_BF16, np.uint16)
    p_i = _full((tp, p_rows, k), -1, np.int64)
    q_rows = (((2.0, 10), (0.0, 11)),) * 3 + (((0.0, 10), (1.0, 11)),)
    p0_rows = (((2.0, 10), (0.0, 11)), ((0.0, 10), (2.0, 11)), ((1.0, 10), (1.0, 11)),
               ((2.0, 10), (0.0, 11)))
    p1_rows = tuple(((0.0, 90 + r * 2), (2.0, 91 + r * 2)) for r in range(rows))
    for r in range(rows):
        for rank, (score, tok) in enumerate(q_rows[r]):
            q_s[rank, r, 0], q_i[rank, r, 0] = bf16([score])[0], tok
        for rank, (score, tok) in enumerate(p0_rows[r]):
            p_s[rank, 2 * r, 0], p_i[rank, 2 * r, 0] = bf16([score])[0], tok
        for rank, (score, tok) in enumerate(p1_rows[r]):
            p_s[rank, 2 * r + 1, 0], p_i[rank, 2 * r + 1, 0] = bf16([score])[0], tok
    temps = [0.0, 0.0, 1.0, 1.0]
    uniforms = [(0.5, 0.2), (0.5, 0.2), (0.9, 0.2), (0.2, 0.2)]
    dec = oracle.verify_k1(q_s, q_i, p_s, p_i, [0, 2, 4, 6], [10] * 4, temps, [1.0] * 4, [2] * 4,
                           list(range(4)), [0] * 4, rows, uniforms=np.array(uniforms, np.float32))
    expected = [list(_dict_oracle(q_rows[r], p0_rows[r], p1_rows[r], 10, temps[r],
                                  float(np.float32(uniforms[r][0])), float(np.float32(uniforms[r][1]))))
                for r in range(rows)]
    assert dec.tolist() == expected


@pytest.mark.parametrize("tp", [1, 2, 4])
@pytest.mark.parametrize("capacity", [1, 4, 16])
@pytest.mark.parametrize("reverse", [False, True])
def test_frozen_probabilistic_draws_across_tp_padding_and_row_maps(oracle, tp, capacity, reverse):
    """tests/ops/test_cuda_speculative.py:133-228 method: exact-bf16 scores on a
    0.25 grid, top_k=6, top_p in {0.6,0.9,1.0}, draws at CDF interval midpoints."""
    rng = random.Random(8149 + 97 * tp + 7 * capacity + int(reverse))
    active = max(1, capacity - 1)
    q = _full((tp, capacity, 20), NAN_BF16, np.uint16)
    qi = _full((tp, capacity, 20), -1, np.int64)
    p = _full((tp, 2 * capacity, 20), NAN_BF16, np.uint16)
    pi = _full((tp, 2 * capacity, 20), -1, np.int64)
    target_rows = list(range(0, 2 * active, 2))
    if reverse:
        target_rows.reverse()
    expected, drafts, draws, temps, top_ps = [], [], [], [], []
    for row, target_row in enumerate(target_rows):
        ids = list(range(8))
        rng.shuffle(ids)
        temperature = (0.5, 1.0, 2.0)[row % 3]
        top_p = (0.6, 0.9, 1.0)[row % 3]
        dists = []
        for phase in range(3):
            pairs = tuple((rng.randrange(-12, 13) / 4, tok) for tok in ids)
            ordered = sorted(pairs, key=lambda it: (-it[0], it[1]))
            probs = _distribution(tuple(ordered[:6]), temperature)
            mass, kept = 0.0, {}
            for tok, prob in probs.items():
                if mass <= top_p:
                    kept[tok] = prob
                mass += prob
            total = sum(kept.values())
            dists.append({tok: v / total for tok, v in kept.items()})
            scores, tokens = (q, qi) if phase == 0 else (p, pi)
            physical = row if phase == 0 else target_row + phase - 1
            for ordinal, (score, tok) in enumerate(pairs):
                rank, local = ordinal % tp, ordinal // tp
                scores[rank, physical, local] = bf16([score])[0]
                tokens[rank, physical, local] = tok
        q_prob, p0_prob, p1_prob = dists
        draft = next(iter(q_prob))
        ratio = min(1.0, p0_prob.get(draft, 0.0) / q_prob[draft])
        accept_draw = 0.125 if ratio > 0.25 else 0.875
        accepted = accept_draw < ratio
        dist = p1_prob if accepted else {t: max(0.0, v - q_prob.get(t, 0.0)) for t, v in p0_prob.items()}
        total = sum(dist.values())
        probs = {t: v / total for t, v in dist.items()}
        tok, prob = max(probs.items(), key=lambda x: x[1])
        cumulative = 0.0
        for cand, value in probs.items():
            if cand == tok:
                break
            cumulative += value
        sample_draw = cumulative + prob / 2
        expected.append([int(accepted), _draw(probs, sample_draw)])
        draws.append((accept_draw, sample_draw))
        drafts.append(draft)
        temps.append(temperature)
        top_ps.append(top_p)
    pad = capacity - active
    dec = oracle.verify_k1(q, qi, p, pi, target_rows + [0] * pad, drafts + [0] * pad,
                           temps + [1.0] * pad, top_ps + [1.0] * pad, [6] * capacity,
                           [0] * capacity, [0] * capacity, active,
                           uniforms=np.array(draws + [(0.0, 0.0)] * pad, np.float32))
    assert dec[:active].tolist() == expected
    assert (dec[active:] == -1).all()


# --------------------------------------------------------------------------- #
# Chain verification and merge_prefix
# --------------------------------------------------------------------------- #
def _sparse_candidates(dist, k=20):
    """Candidate row whose T=1 softmax reproduces `dist` up to bf16 score rounding.

    Rows hold fewer than top_k real candidates, so the checks run with the
    underfilled-row allowance (ops/cuda/sampling/speculative.py:189-207)."""
    scores = np.full(k, NAN_BF16, np.uint16)
    ids = np.full(k, -1, np.int64)
    for slot, (tok, prob) in enumerate(sorted(dist.items(), key=lambda x: -x[1])):
        scores[slot] = bf16([math.log(prob)])[0]
        ids[slot] = tok
    return scores, ids


@pytest.mark.parametrize("depth", [1, 3, 4, 7])
def test_chain_boundaries_and_depths(oracle, depth):
    """tests/generation/test_tp_sampling.py:120-178: draft {1:.8, 2:.2}, target
    {1:.4, 2:.6}, bonus {9:1}; a 0.9 draw rejects at its depth (residual -> 2),
    otherwise every draft is accepted and the bonus is 9."""
    draft_s, draft_i = _sparse_candidates({1: 0.8, 2: 0.2})
    target_s, target_i = _sparse_candidates({1: 0.4, 2: 0.6})
    bonus_s, bonus_i = _sparse_candidates({9: 1.0})
    c = 1
    for accepted in range(depth + 1):
        p_s = np.stack([target_s] * depth + [bonus_s])[None]
        p_i = np.stack([target_i] * depth + [bonus_i])[None]
        decisions = np.empty((depth, c, 2), np.int64)
        for d in range(depth):
            u = 0.9 if d == accepted else 0.1
            decisions[d] = oracle.verify_k1(draft_s[None, None], draft_i[None, None], p_s, p_i, [d],
                                            [1], [1.0], [1.0], [20], [0], [0], 1,
                                            uniforms=np.array([[u, 0.5]], np.float32),
                                            allow_underfilled=True)
        merged = oracle.merge_prefix(decisions, c)
        assert merged.tolist() == [[accepted, 9 if accepted == depth else 2]]


def test_merge_prefix_invalid_and_dead_rows(oracle):
    dec = np.array([[[1, 5], [0, 7], [1, 3], [-1, -1]],
                    [[1, 6], [1, 8], [0, 4], [1, 2]]], np.int64)
    out = oracle.merge_prefix(dec, 3)
    assert out.tolist() == [[2, 6], [0, 7], [1, 4], [-1, -1]]
    assert oracle.merge_prefix(dec, 1).tolist() == [[2, 6], [-1, -1], [-1, -1], [-1, -1]]


def test_verify_from_logits_composes_candidates_verify_merge(oracle):
    rng = np.random.default_rng(5)
    c, depth, v = 3, 2, 500
    logits = bf16(rng.standard_normal((c * (depth + 1), v)) * 3)
    # greedy: draft = target argmax of its row -> accepted; bonus = argmax of next row
    f = oracle.bf16_bits_to_f32(logits)
    argmax = [int(np.lexsort((np.arange(v), -f[r]))[0]) for r in range(c * (depth + 1))]
    drafts = np.array([[argmax[s * (depth + 1) + d] for s in range(c)] for d in range(depth)])
    drafts[1, 2] = (drafts[1, 2] + 1) % v  # sequence 2 rejects at depth 1
    q_s = np.full((depth, c, 20), NAN_BF16, np.uint16)
    q_i = np.full((depth, c, 20), -1, np.int64)
    q_s[:, :, 0] = bf16([1.0])[0]
    q_i[:, :, 0] = drafts
    zeros = np.zeros((depth, c))
    _, _, dec, merged = oracle.verify_from_logits(
        logits, q_s, q_i, drafts, zeros, np.ones((depth, c)), np.ones((depth, c), np.int64),
        zeros.astype(np.int64), zeros.astype(np.int64), c)
    assert merged[0].tolist() == [2, argmax[2]]
    assert merged[1].tolist() == [2, argmax[5]]
    assert merged[2].tolist() == [1, argmax[7]]
