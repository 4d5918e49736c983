"""CPU: the root top-k/top-p sampling oracle (ops/cuda/sampling/topk_topp.py:22-121).

Pins, in order:
* the reference test oracle's known answers (tests/ops/test_cuda_topk_topp_sampling.py:65-91),
  with the explicit uniform it uses;
* the expectations of the reference's CUDA tests (:127-201), which hold for
  any Philox draw: greedy ties, malformed sentinels, grammar underfill owned
  per row, top-p support of one token, determinism in (seed, ordinal);
* a float64 brute force (global top-k, temperature softmax, exclusive-CDF
  top-p, inverse-CDF choice) on random rows with explicit uniforms, skipping
  draws that land within float32 rounding of a CDF boundary.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

NAN = float("nan")


def bf16(x) -> np.ndarray:
    """float -> bf16 bits (RNE); NaN stays NaN."""
    f = np.asarray(x, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), out)


def layout(rows_of_pairs, tp: int, k: int):
    """[(scores, ids) per row] with candidates in rank-major order -> [tp, rows, k]."""
    rows = len(rows_of_pairs)
    scores = np.full((tp, rows, k), NAN, np.float32)
    ids = np.full((tp, rows, k), -1, np.int64)
    for r, (sc, ti) in enumerate(rows_of_pairs):
        for v, (s, i) in enumerate(zip(sc, ti)):
            scores[v // k, r, v % k] = s
            ids[v // k, r, v % k] = i
    return scores, ids


def sample(oracle, rows_of_pairs, *, tp=1, k=20, temperature, top_p, top_k, uniform=None, seed=0,
           ordinal=0, fp16=False, **kw):
    scores, ids = layout(rows_of_pairs, tp, k)
    n = len(rows_of_pairs)
    bits = scores.astype(np.float16).view(np.uint16) if fp16 else bf16(scores)
    full = lambda v, dt: np.full(n, v, dt) if np.isscalar(v) else np.asarray(v, dt)
    return oracle.root_sample(bits, ids, full(temperature, np.float32), full(top_p, np.float32),
                              full(top_k, np.int64), full(seed, np.int64), full(ordinal, np.int64),
                              fp16=fp16, uniforms=None if uniform is None else full(uniform, np.float32),
                              **kw)


def one(oracle, scores, ids, **kw):
    tokens, valid = sample(oracle, [(scores, ids)], **kw)
    return int(tokens[0]), bool(valid[0])


def test_reference_oracle_known_answers(oracle):
    assert one(oracle, [2.0, 4.0, 4.0], [7, 19, 3], temperature=0.0, top_p=0.2, top_k=2, uniform=0.9) == (3, True)
    assert one(oracle, [4.0, NAN], [7, -1], temperature=0.0, top_p=1.0, top_k=20, uniform=0.0) == (7, True)
    args = dict(temperature=1.0, top_k=3)
    assert one(oracle, [3.0, 2.0, 1.0, NAN], [30, 20, 10, -1], top_p=0.5, uniform=0.99, **args) == (30, True)
    assert one(oracle, [3.0, 2.0, 1.0, NAN], [30, 20, 10, -1], top_p=0.7, uniform=0.8, **args) == (20, True)
    bad = dict(temperature=0.0, top_p=1.0, top_k=1, uniform=0.0)
    assert one(oracle, [NAN], [-1], **bad) == (-1, False)
    assert one(oracle, [NAN, 2.0], [4, 7], **bad) == (-1, False)


@pytest.mark.parametrize("fp16", [False, True])
def test_reference_cuda_expectations(oracle, fp16):
    kw = dict(tp=4, k=20, fp16=fp16, seed=0x123456789)
    # greedy tie -> smallest id; a NaN with a real id invalidates its row; no candidates invalid
    rows = [([4.0, 4.0], [19, 3]), ([2.0] + [NAN] * 20, [7] + [-1] * 19 + [8]), ([], [])]
    tokens, valid = sample(oracle, rows, temperature=0.0, top_p=0.9, top_k=20, **kw)
    assert tokens.tolist() == [3, -1, -1] and valid.tolist() == [True, False, False]
    # global top-k across ranks, top-p 0.01 keeps only the best
    cand = ([8.0, 7.0] + [NAN] * 18 + [6.0, 5.0] + [NAN] * 18 + [4.0, 3.0] + [NAN] * 18 + [2.0, 1.0],
            [0, 1] + [-1] * 18 + [2, 3] + [-1] * 18 + [4, 5] + [-1] * 18 + [6, 7])
    tokens, valid = sample(oracle, [cand] * 4, temperature=1.0, top_p=0.01, top_k=4, **kw)
    assert tokens.tolist() == [0] * 4 and valid.all()
    # underfill is owned per row: one candidate per row, top_k 20
    rows = [([2.0], [7]), ([2.0], [8]), ([2.0], [9])]
    tokens, valid = sample(oracle, rows, temperature=0.8, top_p=0.9, top_k=20, allow_underfilled=True,
                           constrained_rows=np.array([1, 0, 1], np.uint8), **kw)
    assert tokens.tolist() == [7, -1, 9] and valid.tolist() == [True, False, True]
    rows[2] = ([2.0] + [NAN] * 20, [9] + [-1] * 19 + [17])  # malformed pair stays an error
    tokens, valid = sample(oracle, rows, temperature=0.8, top_p=0.9, top_k=20, allow_underfilled=True,
                           constrained_rows=np.array([0, 1, 1], np.uint8), **kw)
    assert tokens.tolist() == [-1, 8, -1] and valid.tolist() == [False, True, False]
    # seed/ordinal determinism over equal scores and top_k 2
    kw.pop("seed")
    cand = ([0.0] * 80, list(range(80)))
    first, valid = sample(oracle, [cand] * 128, temperature=0.8, top_p=0.9, top_k=2,
                          seed=np.arange(128) + 0x123456789, ordinal=0, **kw)
    again, _ = sample(oracle, [cand] * 128, temperature=0.8, top_p=0.9, top_k=2,
                      seed=np.arange(128) + 0x123456789, ordinal=0, **kw)
    moved, _ = sample(oracle, [cand] * 128, temperature=0.8, top_p=0.9, top_k=2,
                      seed=np.arange(128) + 0x123456789, ordinal=1, **kw)
    assert valid.all() and np.array_equal(first, again) and set(first.tolist()) <= {0, 1}
    assert (first != moved).any() and set(first.tolist()) == {0, 1}


def test_parameter_domain_fails_closed(oracle):
    cand = [([1.0, 0.5], [3, 4])]
    base = dict(temperature=0.7, top_p=0.9, top_k=2, uniform=0.5)
    assert sample(oracle, cand, **base)[1][0]
    for change in (dict(temperature=NAN), dict(temperature=-0.1), dict(temperature=math.inf),
                   dict(top_p=0.0), dict(top_p=1.5), dict(top_p=NAN), dict(top_k=0), dict(top_k=21),
                   dict(top_k=3), dict(seed=-1), dict(ordinal=-1)):
        tokens, valid = sample(oracle, cand, **{**base, **change})
        assert tokens[0] == -1 and not valid[0], change


def brute_force(pairs, temperature, top_p, top_k, u):
    """float64 restatement of topk_topp.py:58-110 (for comparison, not parity)."""
    best = {}
    for s, i in pairs:
        best[(s, i)] = True
    ordered = sorted(best, key=lambda p: (-p[0], p[1]))[:top_k]
    if temperature == 0.0:
        return ordered[0][1], None
    logits = [s / temperature for s, _ in ordered]
    m = max(logits)
    w = [math.exp(x - m) for x in logits]
    tot = sum(w)
    p = [x / tot for x in w]
    kept, excl = [], 0.0
    for q in p:
        kept.append(q if excl <= top_p else 0.0)
        excl += q
    target = u * sum(kept)
    cum, margin = 0.0, math.inf
    for lane, q in enumerate(kept):
        cum += q
        margin = min(margin, abs(cum - target))
        if cum > target:
            return ordered[lane][1], margin
    return None, margin


@pytest.mark.parametrize("tp,k", [(1, 20), (4, 20), (8, 20), (3, 7)])
def test_against_float64_brute_force(oracle, tp, k):
    rng = np.random.default_rng(tp * 100 + k)
    rows, params = [], []
    for _ in range(200):
        n = int(rng.integers(1, tp * k + 1))
        scores = bf16(rng.normal(0, 2, n).astype(np.float32))
        scores_f = (scores.astype(np.uint32) << 16).view(np.float32)
        ids = rng.choice(50000, n, replace=False)
        if n > 2 and rng.random() < 0.3:  # duplicate (score, id) pairs count once
            scores_f[1], ids[1] = scores_f[0], ids[0]
        rows.append((scores_f.tolist(), ids.tolist()))
        real = len({(s, i) for s, i in zip(scores_f.tolist(), ids.tolist())})
        params.append((float(rng.choice([0.0, 0.5, 1.0, 1.7])), float(rng.choice([0.3, 0.8, 1.0])),
                       int(rng.integers(1, min(real, k) + 1)), float(np.float32(rng.random()))))
    t, p, kk, u = (np.array(x) for x in zip(*params))
    tokens, valid = sample(oracle, rows, tp=tp, k=k, temperature=t, top_p=p, top_k=kk, uniform=u)
    checked = 0
    for r, ((sc, ids), (tt, pp, kq, uu)) in enumerate(zip(rows, params)):
        want, margin = brute_force(list(zip(sc, ids)), tt, pp, kq, uu)
        assert valid[r], r
        if margin is not None and margin < 1e-5:
            continue  # float32 vs float64 rounding decides this draw
        assert tokens[r] == want, (r, tt, pp, kq, uu)
        checked += 1
    assert checked > 150
