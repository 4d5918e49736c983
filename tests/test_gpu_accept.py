"""GPU parity: acceptance kernels against the CPU oracle, bit for bit.

Decisions, accepted lengths, emitted tokens and published candidates must be
identical to the oracle (oracle/cubic_oracle.c) on identical logits and draws.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cubic_serve_amd import sampling

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NAN_BF16 = np.uint16(0x7FC0)


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, device=DEV) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def bf16(values):
    return to_bits(torch.tensor(np.asarray(values, np.float32)).to(torch.bfloat16))


def cuda(values, dtype):
    return torch.tensor(values, dtype=dtype, device=DEV)


# --------------------------------------------------------------------------- #
# candidates
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("rows,width", [(3, 300), (2, 32768), (64, 151936), (5, 70001), (2, 400003)])
def test_candidates_match_oracle(oracle, rows, width):
    print(f"candidates rows={rows} width={width}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + width)
    logits = (torch.randn((rows, width), generator=g) * 3).to(torch.bfloat16)
    bits = to_bits(logits).copy()
    # exact ties across tiles and -0/+0 ties
    bits[0, 5] = bits[0, width - 1] = np.uint16(0x4200)  # 32.0: a tie for the maximum
    bits[0, 17] = np.uint16(0x8000)
    bits[0, 18] = np.uint16(0x0000)
    if rows > 2:
        bits[2, width // 2] = np.uint16(0x7FC0)  # NaN row -> id -2
    # greedy row 1: a tie for the maximum across tiles (lowest id wins)
    bits[1, 7] = bits[1, width - 2] = np.uint16(0x4300)
    if rows > 4:
        # greedy row 4: every value negative but a -0 (id 100) and a +0 (id
        # width - 5); -0 == +0, so the lower id and its own bits are published
        bits[4] = bits[4] | np.uint16(0x8000)
        bits[4, 100] = np.uint16(0x8000)
        bits[4, width - 5] = np.uint16(0x0000)
    if rows > 16:
        # greedy rows 7, 10, 13, 16 inside whole tiles (8 chunks of 2048, a
        # lane holding elements 8 l .. 8 l + 7 of each chunk): a maximum tied
        # within one lane across chunks, within one 32-bit word, at a lane's
        # last element, and a -inf (non-finite row)
        bits[7, 3] = bits[7, 3 + 2048] = np.uint16(0x4400)
        bits[10, 4] = bits[10, 5] = np.uint16(0x4400)
        bits[13, 40 + 7 * 2048 + 7] = np.uint16(0x4400)
        bits[16, 1000] = np.uint16(0xFF80)
    temps = np.array([(0.0 if r % 3 == 1 else 0.7) for r in range(rows)], np.float32)
    owned = max(1, rows - 1)
    count, capacity = 20, 24
    scores = torch.empty((rows, capacity), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((rows, capacity), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    plan = sampling.LocalCandidatePlan(local_logits=from_bits(bits), workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=count, owned_rows=owned)
    for _ in range(2):  # the second launch checks the self-resetting arrival counters
        plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
        torch.cuda.synchronize()
        want_s, want_i = oracle.candidates(bits, temps, count, capacity, owned_rows=owned)
        assert np.array_equal(ids.cpu().numpy(), want_i)
        assert np.array_equal(to_bits(scores), want_s)


@pytest.mark.parametrize("rows,width", [(3, 300), (4, 32768), (64, 151936), (5, 70001)])
def test_fp16_candidates_match_oracle(oracle, rows, width):
    """fp16 logits (local_candidates.py:41): fp16 scores published, fp16 NaN
    padding, non-finite rows (fp16 inf is 0x7C00) give -2, ties by ascending id."""
    print(f"fp16 candidates rows={rows} width={width}", flush=True)
    g = torch.Generator().manual_seed(rows * 11 + width)
    logits = (torch.randn((rows, width), generator=g) * 3).to(torch.float16)
    bits = logits.view(torch.int16).numpy().view(np.uint16).copy()
    bits[0, 5] = bits[0, width - 1] = np.uint16(0x5400)  # 64.0: a tie for the maximum
    bits[0, 17] = np.uint16(0x8000)
    bits[0, 18] = np.uint16(0x0000)
    bits[1, 7] = bits[1, width - 2] = np.uint16(0x5800)  # greedy row: tie across tiles
    if rows > 2:
        bits[2, width // 3] = np.uint16(0x7C00)          # +inf row -> id -2
    if rows > 4:
        bits[4] = bits[4] | np.uint16(0x8000)             # greedy row, all negative but -0/+0
        bits[4, 100] = np.uint16(0x8000)
        bits[4, width - 5] = np.uint16(0x0000)
    if rows > 16:
        # greedy rows 7, 10, 13, 16 inside whole tiles (8 chunks of 2048, a
        # lane holding elements 8 l .. 8 l + 7 of each chunk): a maximum tied
        # within one lane across chunks, within one 32-bit word, at a lane's
        # last element, and a -inf (non-finite row)
        bits[7, 3] = bits[7, 3 + 2048] = np.uint16(0x4400)
        bits[10, 4] = bits[10, 5] = np.uint16(0x4400)
        bits[13, 40 + 7 * 2048 + 7] = np.uint16(0x4400)
        bits[16, 1000] = np.uint16(0xFF80)
    temps = np.array([(0.0 if r % 3 == 1 else 0.7) for r in range(rows)], np.float32)
    count, capacity = 20, 24
    scores = torch.empty((rows, capacity), dtype=torch.float16, device=DEV)
    ids = torch.empty((rows, capacity), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    dev_logits = torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(DEV)
    plan = sampling.LocalCandidatePlan(local_logits=dev_logits, workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=count)
    for _ in range(2):
        plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
        torch.cuda.synchronize()
        want_s, want_i = oracle.candidates(bits, temps, count, capacity, fp16=True)
        assert np.array_equal(ids.cpu().numpy(), want_i)
        assert np.array_equal(scores.cpu().view(torch.int16).numpy().view(np.uint16), want_s)
    if rows > 2:
        assert (ids[2, :count] == -2).all()


def _f32_case(rows, width, seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn((rows, width), generator=g) * 3).numpy().astype(np.float32)
    logits[0, 5] = logits[0, width - 1] = 64.0            # tie for the maximum across tiles
    logits[0, 17], logits[0, 18] = np.float32(-0.0), np.float32(0.0)
    if rows > 1:
        logits[1, 7] = logits[1, width - 2] = 80.0        # greedy row: tie across tiles
    if rows > 2:
        logits[2, width // 3] = np.nan                    # non-finite row -> id -2
    if rows > 4:
        logits[4] = -np.abs(logits[4]) - 1.0             # greedy row: all negative but -0/+0
        logits[4, width // 2], logits[4, width - 5] = np.float32(-0.0), np.float32(0.0)
    if rows > 6:
        logits[6, width - 1] = -np.inf                    # non-finite in the last tile
    if rows > 7:
        logits[7, :] = np.float32(1.5)                    # all equal: lowest ids
    temps = np.array([(0.0 if r % 3 == 1 else 0.7) for r in range(rows)], np.float32)
    return logits, temps


@pytest.mark.parametrize("rows,width,pad", [(3, 300, 0), (5, 4097, 0), (8, 8192, 3), (64, 151936, 0),
                                            (2, 400003, 1), (9, 20, 0)])
def test_f32_candidates_match_oracle(oracle, rows, width, pad):
    """fp32 logits (local_candidates.py:41, SCORE_TYPE 2): fp32 scores published bit
    for bit, fp32 NaN padding, -2 for non-finite rows, ties by ascending id; an odd
    row stride (pad) takes the one-column-per-lane loads."""
    print(f"f32 candidates rows={rows} width={width} pad={pad}", flush=True)
    logits, temps = _f32_case(rows, width, rows * 13 + width)
    count, capacity = min(20, width), 24
    owned = max(1, rows - 1)
    dev_full = torch.zeros((rows, width + pad), dtype=torch.float32, device=DEV)
    dev_full[:, :width] = torch.from_numpy(logits).to(DEV)
    scores = torch.empty((rows, capacity), dtype=torch.float32, device=DEV)
    ids = torch.empty((rows, capacity), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    plan = sampling.LocalCandidatePlan(local_logits=dev_full[:, :width], workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=count, owned_rows=owned)
    want_s, want_i = oracle.candidates_f32(logits, temps, count, capacity, owned_rows=owned)
    for _ in range(2):
        scores.fill_(1.0)
        ids.fill_(7)
        plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), want_i)
        assert np.array_equal(scores.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    if owned > 2:
        assert (ids[2, :count] == -2).all()


@pytest.mark.parametrize("count,capacity,all_random", [(1, 1, False), (7, 64, False), (20, 64, True)])
def test_f32_candidates_counts_offset_all_random(oracle, count, capacity, all_random):
    rows, width, start = 9, 9000, 1000
    logits, temps = _f32_case(rows, width, count * 31 + capacity)
    scores = torch.empty((rows, capacity), dtype=torch.float32, device=DEV)
    ids = torch.empty((rows, capacity), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    plan = sampling.LocalCandidatePlan(local_logits=torch.from_numpy(logits).to(DEV), workspace=ws,
                                       active_rows=rows, visible_width=width, local_count=count,
                                       vocab_start=start, all_random_rows=all_random)
    plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
    torch.cuda.synchronize()
    want_s, want_i = oracle.candidates_f32(logits, temps, count, capacity, all_random=all_random,
                                           vocab_start=start)
    assert np.array_equal(ids.cpu().numpy(), want_i)
    assert np.array_equal(scores.cpu().numpy().view(np.uint32), want_s.view(np.uint32))


def test_f32_candidates_device_metadata_in_graph(oracle):
    """metadata[0] and row_activity read at replay (local_candidates.py:55-70), fp32."""
    rows, width, count = 8, 20000, 20
    logits, temps = _f32_case(rows, width, 99)
    scores = torch.empty((rows, count), dtype=torch.float32, device=DEV)
    ids = torch.empty((rows, count), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    meta = torch.tensor([rows], dtype=torch.int32, device=DEV)
    activity = torch.ones(rows, dtype=torch.bool, device=DEV)
    plan = sampling.LocalCandidatePlan(local_logits=torch.from_numpy(logits).to(DEV), workspace=ws,
                                       active_rows=rows, visible_width=width, local_count=count,
                                       metadata=meta, row_activity=activity)
    full_s, full_i = oracle.candidates_f32(logits, temps, count, count)
    t_dev = torch.from_numpy(temps).to(DEV)
    plan.launch(temperatures=t_dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.launch(temperatures=t_dev)
    for n, act in ((rows, [1] * rows), (5, [1, 0, 1, 1, 0, 1, 1, 1]), (0, [1] * rows)):
        meta[0] = n
        activity.copy_(torch.tensor(act, dtype=torch.bool))
        graph.replay()
        torch.cuda.synchronize()
        got_s, got_i = scores.cpu().numpy().view(np.uint32), ids.cpu().numpy()
        for r in range(rows):
            if r < n and act[r]:
                assert np.array_equal(got_i[r], full_i[r]), (n, r)
                assert np.array_equal(got_s[r], full_s[r].view(np.uint32)), (n, r)
            else:
                assert (got_i[r] == -1).all() and (got_s[r] == 0x7FC00000).all(), (n, r)
    graph.reset()


def test_candidates_all_equal_row_takes_lowest_ids(oracle):
    rows, width = 2, 40000
    bits = np.full((rows, width), np.uint16(0x3F80), np.uint16)  # all 1.0
    temps = np.array([1.0, 0.0], np.float32)
    scores = torch.empty((rows, 20), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((rows, 20), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    plan = sampling.LocalCandidatePlan(local_logits=from_bits(bits), workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=20)
    plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
    want_s, want_i = oracle.candidates(bits, temps, 20, 20)
    assert ids[0].cpu().tolist() == list(range(20))
    assert np.array_equal(ids.cpu().numpy(), want_i)
    assert np.array_equal(to_bits(scores), want_s)


# --------------------------------------------------------------------------- #
# verify_one_draft_candidates: reference known answers
# --------------------------------------------------------------------------- #
def _verify(q, qi, p, pi, target_rows, drafts, temps, top_ps, top_ks, seeds, ordinals, active,
            uniforms=None, allow_underfilled=False, constrained=None):
    q_rows = q.shape[1]
    dec = torch.full((q_rows, 2), 713, dtype=torch.int64, device=DEV)
    sampling.verify_one_draft_candidates(
        q_scores=from_bits(q), q_token_ids=torch.from_numpy(qi).to(DEV), p_scores=from_bits(p),
        p_token_ids=torch.from_numpy(pi).to(DEV), target_rows=cuda(target_rows, torch.int32),
        draft_tokens=cuda(drafts, torch.int64), temperatures=cuda(temps, torch.float32),
        top_ps=cuda(top_ps, torch.float32), top_ks=cuda(top_ks, torch.int64),
        seeds=cuda(seeds, torch.int64), ordinals=cuda(ordinals, torch.int64), decisions=dec,
        active_rows=active,
        uniforms=None if uniforms is None else cuda(np.asarray(uniforms, np.float32), torch.float32),
        allow_underfilled=allow_underfilled,
        constrained_rows=None if constrained is None else cuda(constrained, torch.bool))
    torch.cuda.synchronize()
    return dec.cpu().numpy()


def test_grammar_underfill_known_answer():
    # tests/ops/test_cuda_speculative.py:73-100
    q = np.full((1, 2, 20), NAN_BF16, np.uint16)
    qi = np.full((1, 2, 20), -1, np.int64)
    p = np.full((1, 4, 20), NAN_BF16, np.uint16)
    pi = np.full((1, 4, 20), -1, np.int64)
    q[:, :, 0] = p[:, :, 0] = bf16([1.0])[0]
    qi[:, :, 0] = pi[:, :, 0] = 3
    dec = _verify(q, qi, p, pi, [0, 2], [3, 3], [1.0, 1.0], [1.0, 1.0], [20, 20], [1, 1], [0, 0], 2,
                  uniforms=[[0.5, 0.5]] * 2, allow_underfilled=True, constrained=[True, False])
    assert dec.tolist() == [[1, 3], [-1, -1]]


@pytest.mark.parametrize("source", ["q", "p0", "p1"])
@pytest.mark.parametrize("score,token", [(math.nan, -2), (math.nan, 9), (math.inf, 9), (-math.inf, 9)])
def test_owned_failure_is_not_padding_known_answer(source, score, token):
    # tests/ops/test_cuda_speculative.py:102-131
    q = np.full((4, 4, 20), NAN_BF16, np.uint16)
    qi = np.full((4, 4, 20), -1, np.int64)
    p = np.full((4, 8, 20), NAN_BF16, np.uint16)
    pi = np.full((4, 8, 20), -1, np.int64)
    q[0, :3, 0], qi[0, :3, 0] = bf16([2.0])[0], 10
    p[0, :, 0] = bf16([2.0])[0]
    pi[0, ::2, 0], pi[0, 1::2, 0] = 10, 11
    rows = (4, 2, 0)
    s, i, r = (q, qi, 1) if source == "q" else (p, pi, rows[1] + (source == "p1"))
    s[3, r, 0], i[3, r, 0] = bf16([score])[0], token
    dec = _verify(q, qi, p, pi, (*rows, 0), [10] * 4, [1.0] * 4, [1.0] * 4, [1] * 4, [1] * 4,
                  [0] * 4, 3, uniforms=[[0.5, 0.5]] * 4)
    assert dec.tolist() == [[1, 11], [-1, -1], [1, 11], [-1, -1]]


@pytest.mark.parametrize("tp", [1, 2, 4, 8])
@pytest.mark.parametrize("use_uniforms", [True, False])
def test_random_verify_matches_oracle_bitwise(oracle, tp, use_uniforms):
    """Random candidates (duplicates, padding, poisoned lanes, invalid params)."""
    rng = np.random.default_rng(1000 + tp * 2 + use_uniforms)
    k, q_rows, p_rows = 20, 64, 130
    print(f"verify tp={tp} uniforms={use_uniforms}", flush=True)
    q = bf16(np.round(rng.standard_normal((tp, q_rows, k)) * 8) / 4)
    p = bf16(np.round(rng.standard_normal((tp, p_rows, k)) * 8) / 4)
    qi = rng.integers(0, 40, (tp, q_rows, k)).astype(np.int64)
    pi = rng.integers(0, 40, (tp, p_rows, k)).astype(np.int64)
    # padding tails, some poisoned lanes
    pad_q = rng.random((tp, q_rows, k)) < 0.3
    pad_p = rng.random((tp, p_rows, k)) < 0.3
    q[pad_q], qi[pad_q] = NAN_BF16, -1
    p[pad_p], pi[pad_p] = NAN_BF16, -1
    qi[0, 5, 3] = -2
    p[0, 9, 1] = bf16([math.inf])[0]
    target_rows = rng.integers(-1, p_rows, q_rows).astype(np.int32)
    # mostly the best real q candidate (positive draft probability), else random
    qf = np.where(qi >= 0, torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).float().numpy(), -np.inf)
    flat = qf.transpose(1, 0, 2).reshape(q_rows, -1)
    best = qi.transpose(1, 0, 2).reshape(q_rows, -1)[np.arange(q_rows), flat.argmax(-1)]
    drafts = np.where(rng.random(q_rows) < 0.85, best, rng.integers(0, 40, q_rows))
    temps = rng.choice([0.0, 0.5, 0.7, 1.0, 2.0, 0.7, 1.0, -1.0], q_rows).astype(np.float32)
    top_ps = rng.choice([0.6, 0.9, 1.0, 1.0, 0.9, 0.0], q_rows).astype(np.float32)
    top_ks = rng.choice([1, 2, 6, 20, 20, 6, 21], q_rows).astype(np.int64)
    seeds = rng.integers(-1, 2**40, q_rows).astype(np.int64)
    ordinals = rng.integers(0, 1000, q_rows).astype(np.int64)
    uniforms = rng.random((q_rows, 2)).astype(np.float32) if use_uniforms else None
    active = q_rows - 3
    args = (q, qi, p, pi, target_rows, drafts, temps, top_ps, top_ks, seeds, ordinals, active)
    dec = _verify(*args, uniforms=uniforms, allow_underfilled=bool(tp % 2 == 0))
    want = oracle.verify_k1(q, qi, p, pi, target_rows, drafts, temps, top_ps, top_ks, seeds,
                            ordinals, active, uniforms=uniforms, allow_underfilled=bool(tp % 2 == 0))
    assert np.array_equal(dec, want)
    assert (want[:, 0] >= 0).sum() > 5  # the sweep exercises valid rows


def test_merge_prefix_matches_oracle(oracle):
    rng = np.random.default_rng(4)
    depth, c = 5, 100
    dec = np.stack([rng.integers(0, 2, (depth, c)), rng.integers(0, 50, (depth, c))], -1)
    dec[rng.random((depth, c)) < 0.05] = -1
    out = torch.empty((c, 2), dtype=torch.int64, device=DEV)
    live = torch.tensor([c - 7], dtype=torch.int32, device=DEV)
    sampling.merge_prefix(torch.from_numpy(dec).to(DEV), out, live)
    assert np.array_equal(out.cpu().numpy(), oracle.merge_prefix(dec, c - 7))


# --------------------------------------------------------------------------- #
# fused verify from logits
# --------------------------------------------------------------------------- #
def _fused_case(oracle, c, depth, width, stochastic, seed, use_uniforms=True, live=None, k=20,
                device_live=False):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    rows = c * (depth + 1)
    target = (torch.randn((rows, width), generator=g) * 3).to(torch.bfloat16)
    tbits = to_bits(target)
    temps = np.full((depth, c), 0.7 if stochastic else 0.0, np.float32)
    if stochastic:
        noise = (target.float().reshape(c, depth + 1, width)[:, :depth]
                 + torch.randn((c, depth, width), generator=g)).to(torch.bfloat16)
        qb = to_bits(noise.permute(1, 0, 2).reshape(depth * c, width))
        qs, qid = oracle.candidates(qb, np.full(depth * c, 0.7, np.float32), k)
        q_scores = qs.reshape(depth, c, k)
        q_ids = qid.reshape(depth, c, k)
        # drafts: q's first or second candidate (positive draft probability)
        pick = ((rng.random((depth, c)) < 0.2) & (k > 1)).astype(np.int64)
        drafts = np.take_along_axis(q_ids, pick[..., None], -1)[..., 0]
    else:
        f = oracle.bf16_bits_to_f32(tbits)
        argmax = np.array([int(np.lexsort((np.arange(width), -f[r]))[0]) for r in range(rows)])
        drafts = np.array([[argmax[s * (depth + 1) + d] for s in range(c)] for d in range(depth)])
        miss = rng.random((depth, c)) > 0.7
        drafts = np.where(miss, (drafts + 1) % width, drafts)
        q_scores = np.full((depth, c, k), NAN_BF16, np.uint16)
        q_ids = np.full((depth, c, k), -1, np.int64)
        q_scores[:, :, 0] = bf16([1.0])[0]
        q_ids[:, :, 0] = drafts
    top_ps = np.full((depth, c), 0.9 if stochastic else 1.0, np.float32)
    top_ks = np.full((depth, c), 20 if k == 20 else max(1, k - 2), np.int64)
    seeds = rng.integers(0, 2**40, (depth, c)).astype(np.int64)
    ordinals = rng.integers(0, 10000, (depth, c)).astype(np.int64)
    uniforms = rng.random((depth, c, 2)).astype(np.float32) if use_uniforms else None
    live = c if live is None else live
    plan = sampling.MTPVerifyPlan(
        logits=from_bits(tbits), q_scores=from_bits(q_scores), q_token_ids=torch.from_numpy(q_ids).to(DEV),
        draft_tokens=torch.from_numpy(drafts).to(DEV), temperatures=torch.from_numpy(temps).to(DEV),
        top_ps=torch.from_numpy(top_ps).to(DEV), top_ks=torch.from_numpy(top_ks).to(DEV),
        seeds=torch.from_numpy(seeds).to(DEV), ordinals=torch.from_numpy(ordinals).to(DEV),
        uniforms=None if uniforms is None else torch.from_numpy(uniforms).to(DEV))
    want = oracle.verify_from_logits(tbits, q_scores, q_ids, drafts, temps, top_ps, top_ks, seeds,
                                     ordinals, live, uniforms, count=k)
    for _ in range(2):
        plan.launch(live_rows=live)
        torch.cuda.synchronize()
        assert np.array_equal(plan.candidate_ids.cpu().numpy(), want[1])
        assert np.array_equal(to_bits(plan.candidate_scores), want[0])
        assert np.array_equal(plan.decisions.cpu().numpy(), want[2])
        assert np.array_equal(plan.merged.cpu().numpy(), want[3])
    emitted = plan.emitted.cpu().numpy()
    for s in range(c):
        acc, bonus = want[3][s]
        if acc < 0:
            assert (emitted[s] == -1).all()
        else:
            assert emitted[s, :acc].tolist() == drafts[:acc, s].tolist()
            assert emitted[s, acc] == bonus and (emitted[s, acc + 1:] == -1).all()
    if device_live:
        # one captured launch reading the live count on the device, replayed
        # for several counts (eager work between replays)
        count = torch.tensor([c], dtype=torch.int32, device=DEV)
        plan.launch(live_rows=count)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            plan.launch(live_rows=count)
        for n in (c, live, 1, 0, c - 1):
            count.fill_(n)
            graph.replay()
            torch.cuda.synchronize()
            w = oracle.verify_from_logits(tbits, q_scores, q_ids, drafts, temps, top_ps, top_ks, seeds,
                                          ordinals, n, uniforms, count=k)
            assert np.array_equal(plan.candidate_ids.cpu().numpy(), w[1]), n
            assert np.array_equal(to_bits(plan.candidate_scores), w[0]), n
            assert np.array_equal(plan.decisions.cpu().numpy(), w[2]), n
            assert np.array_equal(plan.merged.cpu().numpy(), w[3]), n
        graph.reset()
    return want


def test_fused_greedy_cfg2_shape(oracle):
    """batch 32, k=1, vocab 151936, ~70% greedy matches."""
    want = _fused_case(oracle, 32, 1, 151936, False, 2)
    assert 0 < (want[3][:, 0] == 1).sum() < 32


def test_fused_stochastic_cfg3_shape(oracle):
    """batch 64, k=3, vocab 151936, T=0.7 top-p 0.9 top-k 20."""
    want = _fused_case(oracle, 64, 3, 151936, True, 3)
    assert (want[3][:, 0] >= 0).mean() > 0.8


@pytest.mark.parametrize("use_uniforms", [True, False])
def test_fused_small_shapes_and_dead_rows(oracle, use_uniforms):
    _fused_case(oracle, 5, 2, 3000, True, 11, use_uniforms=use_uniforms, live=3)
    _fused_case(oracle, 1, 1, 32768, False, 12)


@pytest.mark.parametrize("k", [1, 3, 7, 16])
@pytest.mark.parametrize("stochastic", [True, False])
def test_fused_fewer_candidates(oracle, k, stochastic):
    """Capacity below 20 (verification blocks of 1 to 16 lanes), top_k = k - 2."""
    _fused_case(oracle, 6, 2, 9000, stochastic, 30 + k, k=k)


@pytest.mark.parametrize("stochastic", [True, False])
def test_fused_wide_vocabulary(oracle, stochastic):
    """A vocabulary past 24 tiles of 8 chunks (393216): tiles of up to 16
    chunks per thread, the largest tile-phase variant."""
    _fused_case(oracle, 2, 1, 400003, stochastic, 21)


@pytest.mark.parametrize("stochastic", [True, False])
def test_fused_deep_drafts(oracle, stochastic):
    """k = 5 drafts: depths past the fourth are verified on a second pass of
    the waves, reading their inputs directly rather than from the prefetch."""
    _fused_case(oracle, 3, 5, 5000, stochastic, 13, live=2)


@pytest.mark.parametrize("stochastic", [True, False])
def test_fused_device_live_count_in_one_graph(oracle, stochastic):
    """The live count read on the device when the launch runs (the reference
    composition writes ctx[0] into the sampler metadata, draft_graph.py:
    1046-1067): one captured launch serves every count."""
    _fused_case(oracle, 8, 2, 9000, stochastic, 41, live=5, device_live=True)


def test_candidates_device_metadata_and_activity(oracle):
    """LocalCandidatePlan(metadata=, row_activity=) (local_candidates.py:55-70):
    rows below metadata[0] whose activity flag is set are owned, read at replay."""
    rows, width, count = 8, 20000, 20
    g = torch.Generator().manual_seed(77)
    bits = to_bits((torch.randn((rows, width), generator=g) * 3).to(torch.bfloat16)).copy()
    temps = np.array([0.0, 0.7] * (rows // 2), np.float32)
    scores = torch.empty((rows, count), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((rows, count), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    meta = torch.tensor([rows, 0], dtype=torch.int32, device=DEV)
    activity = torch.ones(rows, dtype=torch.bool, device=DEV)
    plan = sampling.LocalCandidatePlan(local_logits=from_bits(bits), workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=count, metadata=meta,
                                       row_activity=activity)
    full_s, full_i = oracle.candidates(bits, temps, count, count)
    t_dev = torch.from_numpy(temps).to(DEV)
    plan.launch(temperatures=t_dev)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.launch(temperatures=t_dev)
    for n, act in ((rows, [1] * rows), (5, [1, 0, 1, 1, 0, 1, 1, 1]), (0, [1] * rows), (3, [0] * rows)):
        meta[0] = n
        activity.copy_(torch.tensor(act, dtype=torch.bool))
        graph.replay()
        torch.cuda.synchronize()
        got_s, got_i = to_bits(scores), ids.cpu().numpy()
        for r in range(rows):
            if r < n and act[r]:
                assert np.array_equal(got_i[r], full_i[r]) and np.array_equal(got_s[r], full_s[r]), (n, r)
            else:
                assert (got_i[r] == -1).all() and (got_s[r] == NAN_BF16).all(), (n, r)
    graph.reset()


def test_candidates_vocab_shard_offset(oracle):
    """A rank's vocabulary shard: published ids are vocab_start + column
    (LocalCandidatePlan(vocab_start=...), local_candidates.py:25-40)."""
    rows, width, count, start = 3, 5000, 20, 151936 - 5000
    g = torch.Generator().manual_seed(5)
    bits = to_bits((torch.randn((rows, width), generator=g) * 3).to(torch.bfloat16)).copy()
    bits[2, 77] = np.uint16(0x7FC0)
    temps = np.array([0.7, 0.0, 0.7], np.float32)
    scores = torch.empty((rows, count), dtype=torch.bfloat16, device=DEV)
    ids = torch.empty((rows, count), dtype=torch.int64, device=DEV)
    ws = sampling.ShardedSamplingWorkspace(scores, ids, scores, ids)
    plan = sampling.LocalCandidatePlan(local_logits=from_bits(bits), workspace=ws, active_rows=rows,
                                       visible_width=width, local_count=count, vocab_start=start)
    plan.launch(temperatures=torch.from_numpy(temps).to(DEV))
    torch.cuda.synchronize()
    want_s, want_i = oracle.candidates(bits, temps, count, count, vocab_start=start)
    assert np.array_equal(ids.cpu().numpy(), want_i)
    assert np.array_equal(to_bits(scores), want_s)
    assert ids[0].min().item() >= start and (ids[2, :count] == -2).all()


@pytest.mark.parametrize("use_uniforms", [True, False])
def test_speculative_output_follows_the_target_distribution(use_uniforms):
    """Speculative sampling leaves the target distribution unchanged
    (tests/generation/test_tp_sampling.py:199-216): drafts drawn from q
    (0.7 / 0.3), target 0.2 / 0.8; the emitted token -- the draft when
    accepted, the residual sample otherwise -- over 20000 independent rows
    follows the target.  top_k = 2: a row admits exactly its two real
    candidates.  With Philox draws (distinct seeds) this also checks the
    on-device generator."""
    n, k = 20000, 20
    rng = np.random.default_rng(4301)
    q_bits = np.full((1, n, k), NAN_BF16, np.uint16)
    p_bits = np.full((1, 2, k), NAN_BF16, np.uint16)
    q_ids = np.full((1, n, k), -1, np.int64)
    p_ids = np.full((1, 2, k), -1, np.int64)
    q_bits[0, :, :2] = bf16(np.log([0.7, 0.3]))
    p_bits[0, :, :2] = bf16(np.log([0.2, 0.8]))
    q_ids[0, :, :2] = [0, 1]
    p_ids[0, :, :2] = [0, 1]

    def softmax(bits):
        v = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        e = np.exp(v - v.max())
        return e / e.sum()

    q_probs, target = softmax(q_bits[0, 0, :2]), softmax(p_bits[0, 0, :2])
    drafts = (rng.random(n) >= q_probs[0]).astype(np.int64)
    uniforms = rng.random((n, 2)).astype(np.float32) if use_uniforms else None
    seeds = rng.integers(0, 2**40, n).astype(np.int64)
    ordinals = rng.integers(0, 2**20, n).astype(np.int64)
    dec = _verify(q_bits, q_ids, p_bits, p_ids, np.zeros(n, np.int32), drafts,
                  np.ones(n, np.float32), np.ones(n, np.float32), np.full(n, 2, np.int64),
                  seeds, ordinals, n, uniforms=uniforms)
    assert (dec[:, 0] >= 0).all()
    emitted = np.where(dec[:, 0] == 1, drafts, dec[:, 1])
    observed = np.bincount(emitted, minlength=2)[:2] / n
    assert np.abs(observed - target).max() < 0.02, (observed, target)
    # and the drafts alone follow q, not the target (the test is not vacuous)
    assert abs(drafts.mean() - q_probs[1]) < 0.02 and abs(q_probs[1] - target[1]) > 0.4
