"""CPU: the greedy sampler oracle (ops/cuda/sampling/greedy.cu:14-139).

Pins, in order:
* the reference test corpora and their expectations: the cross-M corpus of
  tests/ops/test_cuda_greedy_sampling.py:95-109 (maximum, then the minimum
  token id among equal maxima, over vocab shards), the invalid-parameter
  cases of :179-190 and the qualification fixtures of greedy.py:640-660
  (finite rows, tie rows, a non-finite owned row, an invalid seed);
* a literal restatement of the kernels' scan order (greedy.cu:23-28: strict
  greater-than, or equal with a lower column; finiteness before the mask)
  on tiny rows dense in ties, signed zeros, non-finite values and masks;
* the root's per-candidate loop (greedy.cu:94-98) on tiny gathered blocks
  with padding, malformed sentinels and out-of-vocabulary ids;
* the final guard with each predicate flipped alone.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

NAN = float("nan")


def bits_of(values, fp16: bool) -> np.ndarray:
    a = np.asarray(values, np.float32)
    if fp16:
        return a.astype(np.float16).view(np.uint16)
    u = a.view(np.uint32).astype(np.uint64)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(a), np.uint16(0x7FC0), out)


def values_of(bits, fp16: bool) -> np.ndarray:
    b = np.asarray(bits, np.uint16)
    if fp16:
        return b.view(np.float16).astype(np.float32)
    return (b.astype(np.uint32) << 16).view(np.float32)


def scan_row(vals, mask_row=None, vocab_start=0):
    """Literal greedy_partial scan of one row (single thread, ascending j)."""
    best, best_id, good = -math.inf, None, True
    for j, v in enumerate(vals):
        v = float(v)
        good &= math.isfinite(v)
        if mask_row is not None:
            tok = vocab_start + j
            if not (int(mask_row[tok // 32]) >> (tok % 32)) & 1:
                continue
        if v > best or (v == best and (best_id is None or j < best_id)):
            best, best_id = v, j
    return best, best_id, good


def params(rows, t=0.0, p=0.95, k=20, seed=1, ordinal=0):
    return (np.full(rows, t, np.float32), np.full(rows, p, np.float32), np.full(rows, k, np.int64),
            np.full(rows, seed, np.int64), np.full(rows, ordinal, np.int64))


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("tp", [1, 2, 4])
def test_reference_cross_m_corpus(oracle, fp16, tp):
    """tests/ops/test_cuda_greedy_sampling.py:95-109 and :150-165 (TP shards,
    padded vocab spans, every count and both row orders)."""
    width, vocab = (33, 65) if tp == 4 else (4123, 4123 * tp - 7)
    corpus = ((np.arange(3 * width).reshape(3, width) * 3) % 29 - 14).astype(np.float32)
    reference = []
    for row in range(3):
        cands = []
        for s in range(tp):
            visible = max(0, min(vocab, (s + 1) * width) - s * width)
            if visible:
                v = corpus[row, :visible]
                cands.append((float(v.max()), int(np.argmax(v)) + s * width))
        m = max(c[0] for c in cands)
        reference.append(min(c[1] for c in cands if c[0] == m))
    capacity = 8
    for count in (1, 3, 8):
        for perm in (tuple(r % 3 for r in range(count)), tuple(reversed([r % 3 for r in range(count)]))):
            gathered_s, gathered_i = [], []
            for s in range(tp):
                visible = max(0, min(vocab, (s + 1) * width) - s * width)
                logits = np.full((capacity, visible), NAN, np.float32)
                for dst, src in enumerate(perm):
                    logits[dst] = corpus[src, :visible]
                sc, ids = oracle.greedy_candidates(bits_of(logits, fp16), count, 20, fp16=fp16,
                                                   vocab_start=s * width)
                gathered_s.append(sc)
                gathered_i.append(ids)
            tokens, valid = oracle.greedy_root(np.stack(gathered_s), np.stack(gathered_i),
                                               *params(capacity), active=count, cancel=False,
                                               vocab_size=vocab, fp16=fp16)
            assert tokens.tolist() == [reference[r] for r in perm] + [-1] * (capacity - count)
            assert valid.tolist() == [True] * count + [False] * (capacity - count)
            assert oracle.final_guard(tokens, valid, *params(capacity), active=count, k=20,
                                      vocab_size=vocab)
            # greedy.cu:105-109 parameter predicates (test :179-190)
            for which, value in ((0, 1.0), (1, 0.0), (2, 21), (4, -1)):
                bad = list(params(capacity))
                bad[which] = bad[which].copy()
                bad[which][0] = value
                t2, v2 = oracle.greedy_root(np.stack(gathered_s), np.stack(gathered_i), *bad,
                                            active=count, cancel=False, vocab_size=vocab, fp16=fp16)
                assert t2[0] == -1 and not v2[0]
                assert not oracle.final_guard(t2, v2, *bad, active=count, k=20, vocab_size=vocab)


@pytest.mark.parametrize("case", ["finite", "ties", "nonfinite_owned_shard", "invalid_seed"])
def test_reference_qualification_fixtures(oracle, case):
    """greedy.py:640-660 fixtures on one shard: ((col + 7 row) % 19 - 9);
    ties put 12 at both ends; a NaN at [0, 0]; seed -1 on row 0."""
    capacity, width = 4, 37
    for count in (1, 2, 4):
        cpu = np.full((capacity, width), NAN, np.float32)
        cols = np.arange(width)
        for row in range(count):
            cpu[row] = (cols + row * 7) % 19 - 9
            if case == "ties":
                cpu[row, 0] = cpu[row, width - 1] = 12
        if case == "nonfinite_owned_shard":
            cpu[0, 0] = NAN
        p = list(params(capacity))
        if case == "invalid_seed":
            p[3][0] = -1
        _, _, tokens, valid, final = oracle.greedy_sample(bits_of(cpu, False), *p, active=count,
                                                          cancel=False, k=20, vocab_size=width)
        reject = case in ("nonfinite_owned_shard", "invalid_seed")
        assert final == (not reject)
        if not reject:
            expected = [0 if case == "ties" else int(np.argmax(cpu[r])) for r in range(count)]
            assert tokens.tolist() == expected + [-1] * (capacity - count)
        else:
            assert tokens[0] == -1


@pytest.mark.parametrize("fp16", [False, True])
def test_candidates_match_literal_scan(oracle, fp16):
    rng = np.random.default_rng(7)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, -2.5, 3.0, 65504.0, -65504.0], np.float32)
    for trial in range(300):
        rows, width = int(rng.integers(1, 5)), int(rng.integers(0, 70))
        vals = rng.choice(pool, size=(rows, width))
        if trial % 5 == 0 and width:
            vals[rng.integers(rows), rng.integers(width)] = rng.choice([NAN, math.inf, -math.inf])
        bits = bits_of(vals, fp16)
        vocab_start = int(rng.integers(0, 40))
        mask = None
        if trial % 2:
            words = (vocab_start + width + 31) // 32 + 1
            mask = rng.integers(0, 2**32, size=(rows, words), dtype=np.uint64).astype(np.uint32)
            if trial % 7 == 1:
                mask[:] = 0
        active = int(rng.integers(0, rows + 1))
        k = int(rng.integers(1, 6))
        sc, ids = oracle.greedy_candidates(bits, active, k, fp16=fp16, vocab_start=vocab_start,
                                           token_mask=mask)
        nan_bits = 0x7E00 if fp16 else 0x7FC0
        for r in range(rows):
            best, col, good = scan_row(values_of(bits[r], fp16), None if mask is None else mask[r], vocab_start)
            assert (ids[r, 1:] == -1).all() and (sc[r, 1:] == nan_bits).all()
            if r >= active or width == 0:
                assert ids[r, 0] == -1 and sc[r, 0] == nan_bits
            elif not good:
                assert ids[r, 0] == -2 and sc[r, 0] == nan_bits
            elif col is None or not math.isfinite(best):
                assert ids[r, 0] == -1 and sc[r, 0] == nan_bits
            else:
                assert ids[r, 0] == vocab_start + col
                assert sc[r, 0] == bits[r, col]          # the stored value, sign of zero kept


def literal_root(s, i, t, p, k, seed, ordinal, K, vocab, row, active, cancel):
    if row >= active:
        return (-2 if cancel and row == active else -1), False
    best, best_id, good, real_count = -math.inf, None, True, 0
    for v, tok in zip(s, i):
        v, tok = float(v), int(tok)
        real = math.isfinite(v) and 0 <= tok < vocab
        sentinel = math.isnan(v) and tok == -1
        good &= real or sentinel
        real_count += real
        if real and (v > best or (v == best and tok < best_id)):
            best, best_id = v, tok
    ok = (good and real_count >= 1 and t == 0.0 and math.isfinite(p) and 0.0 < p <= 1.0
          and 1 <= k <= K and seed >= 0 and ordinal >= 0)
    return (best_id if ok else -1), ok


@pytest.mark.parametrize("fp16", [False, True])
def test_root_matches_literal_loop(oracle, fp16):
    rng = np.random.default_rng(11)
    for trial in range(300):
        tp, rows, k = int(rng.integers(1, 5)), int(rng.integers(1, 5)), int(rng.integers(1, 6))
        vocab = 50
        s = rng.choice(np.array([NAN, 0.0, -0.0, 1.0, 2.0, -3.0, math.inf], np.float32), size=(tp, rows, k),
                       p=[.4, .1, .1, .15, .15, .08, .02])
        i = rng.integers(0, vocab, size=(tp, rows, k))
        i[np.isnan(s)] = -1
        if trial % 3 == 0:
            i[rng.integers(tp), rng.integers(rows), rng.integers(k)] = rng.choice([-2, vocab, -1])
        t = rng.choice(np.array([0.0, -0.0, 0.5], np.float32), size=rows)
        p = rng.choice(np.array([0.95, 1.0, 0.0, NAN], np.float32), size=rows, p=[.6, .2, .1, .1])
        kk = rng.choice([1, k, k + 1, 0], size=rows, p=[.3, .5, .1, .1]).astype(np.int64)
        seed = rng.choice([1, 0, -1], size=rows, p=[.6, .3, .1]).astype(np.int64)
        ordn = rng.choice([0, 5, -1], size=rows, p=[.6, .3, .1]).astype(np.int64)
        active, cancel = int(rng.integers(0, rows + 1)), bool(rng.integers(0, 2))
        sbits = bits_of(s, fp16)
        tokens, valid = oracle.greedy_root(sbits, i, t, p, kk, seed, ordn, active=active, cancel=cancel,
                                           vocab_size=vocab, fp16=fp16)
        sv = values_of(sbits, fp16)
        for r in range(rows):
            exp = literal_root(sv[:, r, :].ravel(), i[:, r, :].ravel(), float(t[r]), float(p[r]),
                               int(kk[r]), int(seed[r]), int(ordn[r]), k, vocab, r, active, cancel)
            assert (int(tokens[r]), bool(valid[r])) == exp


def test_final_guard_each_predicate(oracle):
    cap, vocab, K = 6, 100, 20
    base = dict(tokens=np.array([5, 7, 9, -1, -1, -1]), root_valid=np.ones(cap, bool))
    p = params(cap)
    assert oracle.final_guard(base["tokens"], base["root_valid"], *p, active=3, k=K, vocab_size=vocab)
    assert oracle.final_guard(base["tokens"], None, *p, active=3, k=K, vocab_size=vocab)
    cancelled = base["tokens"].copy()
    cancelled[3] = -2
    assert oracle.final_guard(cancelled, base["root_valid"], *p, active=3, k=K, vocab_size=vocab)
    flips = []
    for tok_idx, value in ((0, -1), (0, vocab), (3, 4), (4, -2)):
        t = base["tokens"].copy()
        t[tok_idx] = value
        flips.append((t, base["root_valid"], p))
    rv = base["root_valid"].copy()
    rv[1] = False
    flips.append((base["tokens"], rv, p))
    for which, value in ((0, 2.5), (0, -0.5), (0, NAN), (1, 0.0), (1, 1.5), (2, 0), (2, K + 1),
                         (3, -1), (4, -1)):
        q = [a.copy() for a in p]
        q[which][2] = value
        flips.append((base["tokens"], base["root_valid"], q))
    for t, rv, q in flips:
        assert not oracle.final_guard(t, rv, *q, active=3, k=K, vocab_size=vocab)
    # temperature 2 is admitted by the guard, and only active rows' parameters count
    q = [a.copy() for a in p]
    q[0][2] = 2.0
    q[3][5] = -1
    assert oracle.final_guard(base["tokens"], base["root_valid"], *q, active=3, k=K, vocab_size=vocab)
    for active in (0, cap + 1):
        assert not oracle.final_guard(np.full(cap, -1), None, *p, active=active, k=K, vocab_size=vocab)
